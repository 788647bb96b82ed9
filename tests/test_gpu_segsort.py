"""GPU: the shadow builds' ordering by (major, minor) -- a count per major,
a scatter into the majors' segments and a per-segment bitonic network (the
wave's lanes up to 64 entries, its LDS slice up to 512, one block beyond: in
its LDS up to 8192, in global memory past that) -- builds the same stores as the radix sort (SILI_SEGSORT=0), on
layers whose columns and block columns fall in each of the three cases, and
the results match the oracle."""
import numpy as np
import pytest

from tests.util import assert_close_terms

pytestmark = pytest.mark.gpu


def _designed(rng, n_in, n_out):
    # column 7: every row (> 512: one block's network, in global memory
    # past 8192 rows); columns
    # 100..109: 30 % of the rows each (the wave's LDS network, or one
    # block's); the rest: a few rows each
    rows = []
    for r in range(n_in):
        c = set(rng.choice(n_out, 3, replace=False).tolist())
        c.add(7)
        if rng.random() < 0.3:
            c.update(range(100, 110))
        rows.append(sorted(c))
    ptrs = np.concatenate([[0], np.cumsum([len(r) for r in rows])]).astype(np.int32)
    cols = np.concatenate([np.asarray(r, np.int32) for r in rows])
    w = rng.normal(0, 1, len(cols)).astype(np.float32)
    return ptrs, cols, w


def _block4(rng, n_in, n_out):
    brows, bcols = (n_in + 3) // 4, (n_out + 3) // 4
    br, bc = [], []
    for r in range(brows):
        s = set(rng.choice(bcols, 2, replace=False).tolist())
        s.add(3)  # block column 3 in every block row
        for c in sorted(s):
            br.append(r)
            bc.append(c)
    tiles = rng.integers(0, 256, (len(br), 16)).astype(np.uint8)
    tiles[:, 0] |= 0x10  # every tile holds a live slot
    return np.asarray(br, np.int32), np.asarray(bc, np.int32), tiles


@pytest.mark.parametrize("n_in", [1500, 3000, 9000])
def test_segment_order_equals_sort(hip, monkeypatch, n_in):
    rng = np.random.default_rng(n_in)
    n_out = 4096
    ptrs, cols, w = _designed(rng, n_in, n_out)
    br, bc, tiles = _block4(rng, n_in, n_out)
    layers = {}
    for mode in ("1", "0"):
        monkeypatch.setenv("SILI_SEGSORT", mode)
        L = hip.SparseLinearLayer(n_in, n_out, 4 * (len(cols) + 16 * len(br)) + 4096)
        L.load_weights(ptrs, cols, w)
        L.load_block4_tiles(br, bc, tiles)
        layers[mode] = L
    monkeypatch.delenv("SILI_SEGSORT")
    assert np.array_equal(layers["1"]._store_digest(), layers["0"]._store_digest())
    x = rng.normal(size=(8, n_in)).astype(np.float32)
    ya, yb = layers["1"].forward_dense(x), layers["0"].forward_dense(x)
    np.testing.assert_allclose(ya, yb, rtol=1e-6, atol=1e-6)
    assert len(layers["1"].export_scattered()["val"]) == len(cols)


def test_segment_order_forward_matches_oracle(hip):
    from oracle import HostLayer
    rng = np.random.default_rng(5)
    n_in, n_out = 2600, 512
    ptrs, cols, w = _designed(rng, n_in, n_out)
    L = hip.SparseLinearLayer(n_in, n_out, 4 * len(cols) + 4096)
    L.load_weights(ptrs, cols, w)
    ex = L.export_scattered()
    H = HostLayer(n_in, n_out).load_encoded(ex["row_byte_start"], ex["row_elem_start"], ex["idx"], ex["val"])
    H.set_scales(np.asarray(L.get_value_scales(), np.float32))
    x = rng.normal(size=(16, n_in)).astype(np.float32)
    assert_close_terms(L.forward_dense(x), H.forward_dense(x), H.forward_dense(x, absmode=True), "forward")
