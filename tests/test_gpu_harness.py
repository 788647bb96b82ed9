"""GPU: the reference's callers' exact call sequences replayed on the drop-in
binding, against the oracle after every call.

- FoldedLayer (sili/sparse_rnn.py:1004-1073 construction, :1120 forward,
  :1152 backward, :1206-1212 synaptogenesis): budget n_in*n_out, load_weights
  of scale-divided values, per-row set_value_scale_raw (and, in rank1 mode,
  per-column set_output_scale_raw), set_importance_scale_raw(lr/6),
  equalize_to_capacity(mrw, bpr) (compact_after_build=False: a compacted
  layer has no room left to grow, and synaptogenesis raises there as in the
  reference); forward_dense per suffix and the fold sum; backward_dense(dy
  tiled over the folds, lr, lr_per_row_nnz=True); build_probes(k) +
  n_inputs x synap_step + equalizer_step + zero_accum, the rows' reservations
  checked against their restatement after every sweep.
- SISLDOLayer (sili/sparse_rnn.py:779-803 with _preseed_random_sparse,
  :249-320): load_weights + equalize_to_capacity(per_row); forward_sparse of
  a top-k CSR input (CSR.from_dense, :80-97); backward through
  dense_to_top_k_csr(dy, k) and backward_sparse(x, ..., lr,
  lr_per_row_nnz=True).  The reference's SparseLinearLayer keeps last_input
  only in forward_dense (sili/cpu_backend.cpp:475-492), so after
  forward_sparse last_input is None on both sides and the dense x is passed
  directly, as SISLDOLayer's docstring intends.

The deterministic layer class is used where codes are compared exactly (the
stochastic classes' rounding draws are checked in test_gpu_train.py)."""
import numpy as np
import pytest

import oracle
from oracle import Block4Reservations, HostLayer, ScatteredReservations, block4_row_use, row_content
from train_util import dx_bound, dx_bound_sparse
from util import assert_close_terms

pytestmark = pytest.mark.gpu

FP4_MAX = 6.0


def folded_suffix(rng, n_in, n_out, density, rank1):
    """A suffix layer's absolute CSR and FoldedLayer's scale recipe
    (per_row: row max |w| -> FP4_MAX; rank1: row and column envelopes)."""
    ptrs, cols = [0], []
    for _ in range(n_in):
        k = max(1, int(rng.binomial(n_out, density)))
        cols.extend(np.sort(rng.choice(n_out, size=k, replace=False)).tolist())
        ptrs.append(len(cols))
    ptrs, cols = np.array(ptrs, np.int32), np.array(cols, np.int32)
    vals = rng.normal(0.0, 0.02, len(cols)).astype(np.float32)
    row_of = np.repeat(np.arange(n_in), np.diff(ptrs))
    row_scales = np.ones(n_in, np.float32)
    col_scales = np.ones(n_out, np.float32)
    if rank1:
        col_scales = rng.uniform(0.5, 2.0, n_out).astype(np.float32)
        col_scales[::7] = 1.0  # left at the default, as a fitted envelope may be
        amax = np.zeros(n_in, np.float32)
        np.maximum.at(amax, row_of, np.abs(vals / col_scales[cols]))
        row_scales = np.where(amax > 0, amax / np.float32(FP4_MAX), 1).astype(np.float32)
        combined = row_scales[row_of] * col_scales[cols]
        vals = np.where(combined > 0, vals / combined, vals).astype(np.float32)
    else:
        for r in range(n_in):
            s, e = int(ptrs[r]), int(ptrs[r + 1])
            if e > s:
                m = float(np.abs(vals[s:e]).max())
                if m > 0.0:
                    row_scales[r] = np.float32(m / FP4_MAX)
                    vals[s:e] /= row_scales[r]
    return ptrs, cols, vals, row_scales, col_scales


@pytest.mark.parametrize("batch", [1, 3])
def test_folded_layer_sequence(hip, batch):
    rng = np.random.default_rng(2026 + batch)
    n_in, out_dim, n_folds, lr = 40, 24, 3, 0.05
    n_out = out_dim * n_folds
    mrw = 20
    bits = max(1, n_out - 1).bit_length()
    bpr = mrw * ((bits + 6) // 7) + 4
    layers, hosts, res = {}, {}, {}
    for suffix, rank1 in (("q", False), ("up", True)):
        ptrs, cols, vals, rs, cs = folded_suffix(rng, n_in, n_out, 0.12, rank1)
        L = hip.SparseLinearLayerDeterministic(n_in, n_out, n_in * n_out, 4)
        L.load_weights(ptrs, cols, vals)
        for r in range(n_in):
            if rs[r] != 1.0:
                L.set_value_scale_raw(r, float(rs[r]))
        for c in range(n_out):
            if cs[c] != 1.0:
                L.set_output_scale_raw(c, float(cs[c]))
        for r in range(n_in):
            L.set_importance_scale_raw(r, lr / FP4_MAX)
        L.equalize_to_capacity(mrw, bpr)
        H = HostLayer(n_in, n_out).load_csr(ptrs, cols, w=vals)
        S = ScatteredReservations(n_in, n_in * n_out)
        S.load(*row_content(H.row_byte_start, H.row_elem_start)).equalize_to_capacity(mrw, bpr)
        res[suffix] = S
        H.set_scales(rs, cs)
        # set_output_scale_raw marks the output scales trainable
        H.output_scale_trainable = bool(rank1)
        H.importance_scale = np.full(n_in, np.float32(lr / FP4_MAX), np.float32)
        H.out_deg = np.bincount(cols, minlength=n_out).astype(np.int32)
        H.acc = (np.zeros(n_in, np.float32), np.zeros(n_out, np.float32))
        # the block4 store as the constructor leaves it: nothing reserved;
        # promotions grow their rows, the update's write-back evicts
        H.b4res = Block4Reservations(n_in, n_in * n_out)
        H.b4_flags = np.zeros(1, np.uint8)
        layers[suffix], hosts[suffix] = L, H
    n_tiles = {s: 0 for s in layers}
    for step in range(9):
        what = f"B{batch} step {step}"
        x = rng.normal(size=(batch, n_in)).astype(np.float32)
        parts, want, bound = [], 0, 0
        for s, L in layers.items():
            H = hosts[s]
            parts.append(L.forward_dense(x))
            want = want + H.forward_dense(x).astype(np.float64)
            bound = bound + H.forward_dense(x, absmode=True).astype(np.float64)
        raw = sum(parts)
        summed = raw.reshape(batch, n_folds, out_dim).sum(axis=1)
        assert_close_terms(summed, want.reshape(batch, n_folds, out_dim).sum(axis=1),
                           bound.reshape(batch, n_folds, out_dim).sum(axis=1), what + ": folded forward")
        dy = rng.normal(size=(batch, out_dim)).astype(np.float32)
        dy_raw = np.tile(dy.reshape(batch, 1, out_dim), (1, n_folds, 1)).reshape(batch, n_out).astype(np.float32)
        for s, L in layers.items():
            H = hosts[s]
            b = dx_bound(H, dy_raw, lr)
            dxg = L.backward_dense(dy_raw, lr, lr_per_row_nnz=True)
            dxh, _, _ = H.backward_train(x, dy_raw, lr, lr_per_row_nnz=True, acc=H.acc)
            assert np.array_equal(L.export_scattered()["val"], H.val[:H.nnz]), f"{what} {s}: value bytes"
            assert_close_terms(dxg, dxh, b, f"{what} {s}: dx")
            if batch == 1:
                assert np.array_equal(L.get_value_scales(), H.value_scale), f"{what} {s}: value_scale"
            else:
                np.testing.assert_allclose(L.get_value_scales(), H.value_scale, rtol=1e-5, atol=0)
            assert_close_terms(L.neuron_input_accum, H.acc[0], H.acc[0], f"{what} {s}: acc_in")
            assert_close_terms(L.neuron_grad_accum, H.acc[1], H.acc[1], f"{what} {s}: acc_grad")
            same_block4(L, H, f"{what} {s}")
        if step % 3 == 2:
            # FoldedLayer.synaptogenesis(k, importance_cutoff, max_row_weights)
            for s, L in layers.items():
                H = hosts[s]
                ai, ag = np.array(L.neuron_input_accum), np.array(L.neuron_grad_accum)
                L.build_probes(8)
                H.build_probes(ai, ag, 8)
                pr, pc, pv = L.get_probes()
                assert np.array_equal(pr, H.probes[0][:H.probe_nnz]) and \
                    np.array_equal(pc, H.probes[1][:H.probe_nnz]), f"{what} {s}: probes"
                S = res[s]
                for _ in range(L.n_inputs):
                    assert L.synap_step(0.6, mrw) == H.synap_step(0.6, mrw, reservations=S), f"{what} {s}: synap_step"
                L.equalizer_step()
                S.equalizer_step()
                # equalizer_step steps the block4 store's rows too
                H.b4res.equalize_step(*block4_row_use(n_in, H.tile_br, H.tile_bc, H.tiles[:16 * H.n_tiles],
                                                       H.b4_flags[:H.n_tiles]))
                L.zero_accum()
                H.acc[0][:] = 0
                H.acc[1][:] = 0
                e = L.export_scattered()
                assert np.array_equal(e["row_elem_start"], H.row_elem_start), f"{what} {s}: structure"
                assert np.array_equal(e["idx"], H.idx[:len(e["idx"])]), f"{what} {s}: index bytes"
                assert np.array_equal(e["val"], H.val[:len(e["val"])]), f"{what} {s}: value bytes"
                assert np.array_equal(L.out_degree, H.out_deg), f"{what} {s}: out_degree"
                assert not np.any(L.neuron_input_accum) and not np.any(L.neuron_grad_accum)
                lay = L.export_layout()
                want = S.layout(*row_content(H.row_byte_start, H.row_elem_start))
                assert all(np.array_equal(lay[k], want[k]) for k in want), f"{what} {s}: reservations"
                same_block4(L, H, f"{what} {s} synaptogenesis")
                n_tiles[s] = max(n_tiles[s], H.n_tiles)
    assert max(n_tiles.values()) > 0, "no tile was promoted"
    assert sum(h.b4_counters[0] for h in hosts.values()) > 0, "the update's write-back evicted nothing"


def same_block4(L, H, what):
    """Tiles, their encoding, the block4 reservations and Block4View's
    counters as the oracle holds them."""
    from train_util import check_b4_reservations
    b = L.export_block4()
    assert np.array_equal(b["br"], H.tile_br) and np.array_equal(b["bc"], H.tile_bc), what + ": tiles"
    assert np.array_equal(b["tiles"], H.tiles[:16 * len(b["br"])]), what + ": tile bytes"
    check_b4_reservations(L, H, what)
    v = L.block4
    assert v.alloc_bytes == sum(H.b4res.ta), what + ": Block4View.alloc_bytes"
    assert (v.dropped_growth_events, v.row_merge_overflow_events, v.row_merge_overflow_bytes_dropped) == \
        (H.b4res.dropped, H.b4_counters[1], H.b4_counters[2]), what + ": Block4View counters"


def test_sisldo_layer_sequence(hip):
    rng = np.random.default_rng(77)
    n_in, n_out, max_weights, p = 64, 96, 64 * 12, 0.1
    per_row = max(2, max_weights // n_in)
    k = max(1, min(n_out, per_row // 2))
    ptrs = np.arange(n_in + 1, dtype=np.int32) * k
    cols = np.concatenate([np.sort(rng.choice(n_out, size=k, replace=False)) for _ in range(n_in)]).astype(np.int32)
    vals = (rng.standard_normal(n_in * k) / np.sqrt(k)).astype(np.float32)
    L = hip.SparseLinearLayer(n_in, n_out, max_weights, 4)
    L.load_weights(ptrs, cols, vals)
    L.equalize_to_capacity(per_row)
    H = HostLayer(n_in, n_out).load_csr(ptrs, cols, w=vals)
    H.out_deg = np.bincount(cols, minlength=n_out).astype(np.int32)
    lr = 0.02
    for step in range(4):
        what = f"step {step}"
        B = 1 + step % 2
        xd = rng.normal(size=(B, n_in)).astype(np.float32)
        kx = max(1, int(n_in * p))
        xp, xi, xv = hip.dense_to_top_k_csr(xd, kx, 4)
        op, oi, ov = oracle.dense_to_top_k_csr(xd, kx)
        assert np.array_equal(xp, op) and np.array_equal(xi, oi) and np.array_equal(xv, ov), what + ": x top-k"
        y = L.forward_sparse(xp, xi, xv, B)
        assert_close_terms(y, H.forward_sparse(xp, xi, xv, B), H.forward_sparse(xp, xi, xv, B, absmode=True),
                           what + ": forward_sparse")
        assert L.last_input is None
        # the dense input the CSR came from (the entries top-k kept)
        x = np.zeros((B, n_in), np.float32)
        for b in range(B):
            x[b, xi[xp[b]:xp[b + 1]]] = xv[xp[b]:xp[b + 1]]
        dy = rng.normal(size=(B, n_out)).astype(np.float32)
        kd = max(1, int(dy.shape[1] * 0.03))
        dp, di, dv = hip.dense_to_top_k_csr(dy, kd, 4)
        gp, gi, gv = oracle.dense_to_top_k_csr(dy, kd)
        assert np.array_equal(dp, gp) and np.array_equal(di, gi) and np.array_equal(dv, gv), what + ": dy top-k"
        dense = np.zeros((B, n_out), np.float32)
        for b in range(B):
            dense[b, di[dp[b]:dp[b + 1]]] = dv[dp[b]:dp[b + 1]]
        bound = dx_bound_sparse(H, dense, lr)
        dxg = L.backward_sparse(x, dp, di, dv, B, lr, lr_per_row_nnz=True)
        dxh, _, _ = H.backward_sparse_train(x, dp, di, dv, B, lr, lr_per_row_nnz=True)
        # the sparse-gradient update rounds to nearest in every layer class
        assert np.array_equal(L.export_scattered()["val"], H.val[:H.nnz]), what + ": value bytes"
        assert_close_terms(dxg, dxh, bound, what + ": dx")
