"""GPU: the synaptogenesis step's key orderings (candidate keys, inserted
windows, the final scattered set) by a count per major and per-segment
bitonic networks -- the wave's lanes up to 64 entries, its LDS up to 512, one
block beyond 512, in its LDS up to 8192 and in global memory past that -- leave the same layer and statistics as the
device radix sort (SILI_KEYORDER=0) and as the oracle, on a layer and
candidate list designed to put segments in each of the three cases, with
repeated candidates (equal keys, ordered by list position) and empty
entries."""
import numpy as np
import pytest

from oracle import HostLayer
from tests.test_gpu_synapto import assert_same_structure

pytestmark = pytest.mark.gpu


def _designed(rng, n_in, n_out):
    # row 5: 3600 columns (final set > 512: global-memory network); rows
    # 10..19: 400 each (LDS network); the rest: a few each (lanes)
    rows = []
    for r in range(n_in):
        if r == 5:
            c = rng.choice(n_out, 3600, replace=False)
        elif 10 <= r < 20:
            c = rng.choice(n_out, 400, replace=False)
        else:
            c = rng.choice(n_out, 4, replace=False)
        rows.append(np.sort(c))
    ptrs = np.concatenate([[0], np.cumsum([len(r) for r in rows])]).astype(np.int32)
    cols = np.concatenate(rows).astype(np.int32)
    q = rng.normal(0, 2, len(cols)).astype(np.float32)
    return ptrs, cols, q, np.ones(len(cols), np.float32)


def _candidates(rng, n_in, n_out):
    # row 7: 2600 distinct columns, so more than 512 candidate keys and, once
    # inserted, more than 512 window entries in block row 1; row 11: 300
    # (LDS); 3000 spread out; then 800 repeats of earlier candidates and 6000
    # of row 7's (its candidate keys past 8192: the global-memory network)
    r7 = np.full(2600, 7)
    c7 = rng.choice(n_out, 2600, replace=False)
    r11 = np.full(300, 11)
    c11 = rng.choice(n_out, 300, replace=False)
    rs, cs = rng.integers(0, n_in, 3000), rng.integers(0, n_out, 3000)
    cr = np.concatenate([r7, r11, rs]).astype(np.int32)
    cc = np.concatenate([c7, c11, cs]).astype(np.int32)
    rep = rng.integers(0, len(cr), 800)
    rep7 = rng.integers(0, 2600, 6000)
    cr = np.concatenate([cr, cr[rep], np.full(6000, 7), [-1, n_in]]).astype(np.int32)
    cc = np.concatenate([cc, cc[rep], c7[rep7], [0, 0]]).astype(np.int32)
    perm = rng.permutation(len(cr))
    cv = rng.normal(0, 0.5, len(cr)).astype(np.float32)
    return cr[perm], cc[perm], cv[perm]


@pytest.mark.parametrize("frac", [0.3, 0.9])
def test_key_order_equals_sort_and_oracle(hip, monkeypatch, frac):
    rng = np.random.default_rng(int(frac * 10))
    n_in, n_out = 600, 4096
    ptrs, cols, q, imp = _designed(rng, n_in, n_out)
    cr, cc, cv = _candidates(rng, n_in, n_out)
    res = {}
    for mode in ("1", "0"):
        monkeypatch.setenv("SILI_KEYORDER", mode)
        L = hip.SparseLinearLayer(n_in, n_out, 4 * (len(cols) + len(cr)) + 4096)
        L.load_weights_with_importance(ptrs, cols, q, imp)
        st = L.synapto_step(frac, cr, cc, cv)
        res[mode] = (L, st)
    monkeypatch.delenv("SILI_KEYORDER")
    (La, sa), (Lb, sb) = res["1"], res["0"]
    assert sa == sb
    assert sa["n_grown"] > 512 and sa["n_promoted_tiles"] > 0
    assert np.array_equal(La._store_digest(), Lb._store_digest())
    H = HostLayer(n_in, n_out).load_csr(ptrs, cols, w=q, imp=imp)
    out, so = H.synapto_step(frac, cr, cc, cv)
    assert sa == so
    assert_same_structure(La, out, f"key order, frac {frac}")
