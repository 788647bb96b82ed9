"""CPU: the bulk synaptogenesis step of the oracle.

The selection policy (k smallest |dec*S|, ties by (row, col); regrow at the
first valid host candidates) has no reference counterpart; its structural
rules are pinned against the reference's own primitives (golden promote /
demote sequences), the rest by invariants."""
import os

import numpy as np
import pytest

from oracle import HostLayer
from sili__new_amd.codec import fp4_decode_np, fp4_encode_np
from sili__new_amd.synth import make_config

G = np.load(os.path.join(os.path.dirname(__file__), "golden", "golden.npz"))


def _abs_eq(H, prefix):
    p, ix, w, imp = H.absolute()
    assert np.array_equal(p, G[prefix + "_abs_ptrs"])
    assert np.array_equal(ix, G[prefix + "_abs_idx"])
    assert np.array_equal(w.view(np.uint32), G[prefix + "_abs_w"].view(np.uint32))
    assert np.array_equal(imp.view(np.uint32), G[prefix + "_abs_imp"].view(np.uint32))


def test_prune_then_promote_matches_reference_primitives():
    pc = G["promote_in"]
    ptrs, cols = pc[:9], pc[9:]
    H = HostLayer(8, 12).load_csr(ptrs, cols, w=G["promote_w"], imp=G["promote_imp"])
    out, st = H.synapto_step(0.2, [2], [3], [3.0], [0.5])
    assert st["n_pruned"] == 1 and st["n_grown"] == 1 and st["n_promoted_tiles"] == 1
    _abs_eq(out, "promote")
    assert np.array_equal(out.tile_br, G["promote_br"]) and np.array_equal(out.tile_bc, G["promote_bc"])
    assert np.array_equal(out.tiles[:16 * out.n_tiles], G["promote_tiles"])


def test_prune_then_demote_matches_reference_primitives():
    dm = G["dm_in"]
    H = HostLayer(8, 8).load_csr(dm[:9], dm[9:], w=G["dm_w"]).load_tiles([0], [0], G["dm_tile"])
    # regrow candidates are all invalid: the just-pruned positions and a stored one
    out, st = H.synapto_step(2 / 6, [0, 2, 0], [0, 1, 6], [1.0, 1.0, 1.0])
    assert st["n_pruned"] == 2 and st["n_grown"] == 0 and st["n_demoted_tiles"] == 1 and st["n_tiles"] == 0
    _abs_eq(out, "dm")
    assert np.array_equal(out.val[:out.nnz], G["dm_val"])
    assert np.array_equal(out.idx[:out.index_bytes], G["dm_idx"])


def _synapses(H):
    """(key bits |w|, row, col) of every stored synapse."""
    p, ix, w, _ = H.absolute()
    rows = np.repeat(np.arange(H.n_in), np.diff(p))
    W = H.dense()
    true = W[rows, ix]
    return np.abs(true).view(np.uint32), rows, ix


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_bulk_step_invariants(seed):
    wl = make_config(3, scale=0.0625)
    H = HostLayer(wl.n_in, wl.n_out).load_tiles(wl.tile_br, wl.tile_bc, wl.tile_bytes).set_scales(wl.value_scale)
    # a scattered part too: every row gets a few synapses outside the tiles
    rng = np.random.default_rng(seed)
    cover = np.zeros((wl.n_in, wl.n_out), bool)
    for br, bc in zip(wl.tile_br, wl.tile_bc):
        cover[br * 4:br * 4 + 4, bc * 4:bc * 4 + 4] = True
    mask = (rng.random((wl.n_in, wl.n_out)) < 0.01) & ~cover
    ptrs = np.concatenate([[0], np.cumsum(mask.sum(1))]).astype(np.int32)
    cols = np.nonzero(mask)[1].astype(np.int32)
    q = rng.normal(0, 2, len(cols)).astype(np.float32)
    # nonzero importance keeps every synapse live through promotion (a
    # promoted byte of 0 is an empty tile slot)
    H.load_csr(ptrs, cols, w=q, imp=np.ones(len(cols), np.float32))
    keys, rows, cols_all = _synapses(H)
    N = len(keys)
    # k = llround(prune_frac * N) with prune_frac held as float32
    k = int(np.floor(float(np.float32(0.01)) * N + 0.5))
    cr = rng.integers(0, wl.n_in, 3 * k + 16).astype(np.int32)
    cc = rng.integers(0, wl.n_out, 3 * k + 16).astype(np.int32)
    cv = rng.normal(0, 0.01, len(cr)).astype(np.float32)
    out, st = H.synapto_step(0.01, cr, cc, cv)
    assert st["n_prune_target"] == k and st["n_pruned"] == k and st["n_grown"] == k
    keys2, rows2, cols2 = _synapses(out)
    # nnz conserved (every regrown synapse is live: default importance code 1)
    assert len(keys2) == N
    # the pruned set is exactly the k smallest (|w| bits, row, col)
    order = np.lexsort((cols_all, rows, keys))
    pruned = set(zip(rows[order[:k]].tolist(), cols_all[order[:k]].tolist()))
    before = set(zip(rows.tolist(), cols_all.tolist()))
    after = set(zip(rows2.tolist(), cols2.tolist()))
    assert not (pruned & after)
    assert before - pruned <= after
    grown = after - (before - pruned)
    assert len(grown) == k
    # regrown synapses are the first valid candidates, in list order
    seen, want = set(), []
    for r, c in zip(cr.tolist(), cc.tolist()):
        if len(want) == k:
            break
        if (r, c) in before or (r, c) in seen:
            continue
        seen.add((r, c))
        want.append((r, c))
    assert grown == set(want)
    # their codes: fp4_encode(v / S)
    W2 = out.dense()
    for i, (r, c) in enumerate(zip(cr.tolist(), cc.tolist())):
        if (r, c) in grown:
            s = np.float32(wl.value_scale[r])
            code = fp4_encode_np(np.array([np.float32(cv[i]) / s], np.float32))[0]
            assert W2[r, c].view(np.uint32) == (fp4_decode_np(code) * s).astype(np.float32).view(np.uint32)
    # structure: rows sorted and unique; every surviving tile that lost a
    # slot still holds >= 2 live slots
    cdec = out.decode_cols()
    for r in range(out.n_in):
        seg = cdec[int(out.row_elem_start[r]):int(out.row_elem_start[r + 1])]
        assert np.all(np.diff(seg) > 0)
    live = (out.tiles[:16 * out.n_tiles].reshape(-1, 16) != 0).sum(1)
    assert np.all(live >= 2)


def test_tie_break_by_row_then_col():
    # all |w| equal: the first k synapses in (row, col) order are pruned
    H = HostLayer(4, 6).load_csr([0, 2, 4, 5, 6], [1, 3, 0, 5, 2, 4], w=[1.0, -1.0, 1.0, 1.0, -1.0, 1.0])
    out, st = H.synapto_step(0.5, [], [], [])
    assert st["n_pruned"] == 3 and st["n_grown"] == 0
    p, ix, _, _ = out.absolute()
    assert p.tolist() == [0, 0, 1, 2, 3] and ix.tolist() == [5, 2, 4]
