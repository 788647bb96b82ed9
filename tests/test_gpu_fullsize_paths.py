"""GPU parity at full size on the paths bench.py times, against the CPU
oracle on the same seeded inputs:

- config 3 (block4, 16384^2, 503,316 tiles, batch 256): forward, grad-input
  with the accumulators, and the sampled grad-W of every slot
  (linear_disldo.hpp:137-339,962-1951);
- config 3's bulk synaptogenesis step at 8,053,056 slots, the first two steps
  bench.py times (prune 80,531, regrow, rebuild): structure byte for byte and
  the step statistics against oracle_synapto_step, then forward and
  grad-input on the rebuilt stores; and the tile merge of the rebuild against
  the full sort, on the internal stores' digests (shadows, work items,
  permutations included);
- config 4's gate-shaped (5120 x 1,310,720) and down-shaped (32768 x 204,800)
  layers at batches 8 and 128 (stream kernels with column blocks, the
  staged-input gather), on sampled batch rows: each output row depends on its
  own input row only;
- value/output scales of rank 3 and 4 (set_scale_rank, cpu_backend.cpp:466)
  through the dense forward at every kernel family's batch, grad-input and
  grad-W, against the closed form S(r, c) = sum_k vs[r, k] os[c, k]
  (delta_csr_types.hpp:1235-1240) on a dense fp64 matrix of the decoded
  codes; and through the sparse-input forward (by push and by gather) and
  the sparse-gradient dx, which read component 0 of each scale only,
  vs[r, 0] * os[c, 0] (sisldo_ops.hpp:302-306,518-529,689-698), against the
  same closed form and the oracle; on a layer with scattered synapses and
  block4 tiles.
"""
import numpy as np
import pytest

from oracle import HostLayer
from sili__new_amd.synth import SEED0, Stream, make_config
from tests.test_gpu_synapto import assert_same_structure
from tests.util import assert_close_terms, gpu_layer, host_layer

pytestmark = pytest.mark.gpu

T = 16  # oracle threads (the GPU box's host share)


@pytest.fixture(scope="module")
def c3():
    wl = make_config(3)
    assert len(wl.tile_br) == 503316 and wl.batch == 256
    return wl


def test_config3_full_size_fwd_gradin_gradw(hip, c3):
    wl = c3
    H = host_layer(wl)
    L = gpu_layer(hip, wl)
    ex = L.export_block4()
    assert np.array_equal(ex["br"], H.tile_br) and np.array_equal(ex["bc"], H.tile_bc)
    assert np.array_equal(ex["tiles"], H.tiles[:16 * H.n_tiles])
    assert np.array_equal(ex["bidx"], H.bidx[:len(ex["bidx"])])
    y = L.forward_dense(wl.x)
    assert_close_terms(y, H.forward_dense(wl.x, threads=T), H.forward_dense(wl.x, absmode=True, threads=T),
                       "c3 fwd")
    del y
    dx = L.backward_dense(wl.g, 0.0)
    dx_o, ai_o, ag_o = H.backward_dense(wl.x, wl.g, threads=T)
    assert_close_terms(dx, dx_o, H.backward_dense(wl.x, wl.g, absmode=True, threads=T)[0], "c3 dx")
    assert_close_terms(L.neuron_input_accum, ai_o, ai_o, "c3 acc_in")
    assert_close_terms(L.neuron_grad_accum, ag_o, ag_o, "c3 acc_grad")
    del dx, dx_o
    gs, gb = L.sampled_gradw(wl.x, wl.g)
    assert len(gs) == 0 and len(gb) == 16 * 503316
    gb_o = H.sampled_gradw(wl.x, wl.g, threads=T)[1]
    assert_close_terms(gb, gb_o, H.sampled_gradw(wl.x, wl.g, absmode=True, threads=T)[1], "c3 grad-W")


def _bench_candidates(wl, i):
    """bench.py time_synapto's candidates of step i (step 0: the config's)."""
    if i == 0:
        return wl.cand_r, wl.cand_c, wl.cand_v
    m = len(wl.cand_r)
    st = Stream(SEED0 + 3, 100 + i)
    return (st.integers(m, wl.n_in).astype(np.int32), st.integers(m, wl.n_out).astype(np.int32),
            Stream(SEED0 + 3, 200 + i).normal(m, 0.01))


def _c3_synapto_layer(hip, wl):
    L = hip.SparseLinearLayer(wl.n_in, wl.n_out, 16 * len(wl.tile_br) + 1024)
    L.load_block4_tiles(wl.tile_br, wl.tile_bc, wl.tile_bytes)
    L.set_value_scales(wl.value_scale)
    return L


def test_config3_synapto_full_size(hip, c3):
    wl = c3
    H = host_layer(wl)
    L = _c3_synapto_layer(hip, wl)
    for i in range(2):
        cr, cc, cv = _bench_candidates(wl, i)
        st = L.synapto_step(0.01, cr, cc, cv)
        H, st_o = H.synapto_step(0.01, cr, cc, cv)
        assert st == st_o, i
        assert st["n_pruned"] == 80531 and st["n_grown"] == 80531, st
        assert_same_structure(L, H, f"c3 synaptogenesis step {i}")
    # the rebuilt shadows serve the gathers
    x, g = wl.x[:64], wl.g[:64]
    assert_close_terms(L.forward_dense(x), H.forward_dense(x, threads=T), H.forward_dense(x, absmode=True, threads=T),
                       "c3 fwd after synaptogenesis")
    dx = L.backward_dense(g, 0.0)
    assert_close_terms(dx, H.backward_dense(x, g, threads=T)[0], H.backward_dense(x, g, absmode=True, threads=T)[0],
                       "c3 dx after synaptogenesis")


def test_config3_synapto_tile_merge_equals_sort(hip, c3, monkeypatch):
    """The rebuild merges the step's two tile runs (survivors in store order,
    promoted windows in window order); SILI_TILE_MERGE=0 sorts them.  Both
    must build identical stores, step after step."""
    wl = c3
    La, Lb = _c3_synapto_layer(hip, wl), _c3_synapto_layer(hip, wl)
    for i in range(3):
        cr, cc, cv = _bench_candidates(wl, i)
        monkeypatch.delenv("SILI_TILE_MERGE", raising=False)
        sa = La.synapto_step(0.01, cr, cc, cv)
        monkeypatch.setenv("SILI_TILE_MERGE", "0")
        sb = Lb.synapto_step(0.01, cr, cc, cv)
        monkeypatch.delenv("SILI_TILE_MERGE")
        assert sa == sb, i
        assert sa["n_promoted_tiles"] > 0, sa
        assert np.array_equal(La._store_digest(), Lb._store_digest()), f"step {i}"


@pytest.mark.parametrize("knob", ["SILI_SEGSORT", "SILI_KEYORDER"])
def test_config3_synapto_segment_order_equals_sort(hip, c3, monkeypatch, knob):
    """The shadow builds (SILI_SEGSORT) and the step's candidate, window and
    final-set keys (SILI_KEYORDER) are ordered by a count per major and a
    per-segment network by default; =0 sorts the keys.  The load and three
    bulk steps give identical stores either way."""
    wl = c3
    monkeypatch.setenv(knob, "1")
    La = _c3_synapto_layer(hip, wl)
    monkeypatch.setenv(knob, "0")
    Lb = _c3_synapto_layer(hip, wl)
    assert np.array_equal(La._store_digest(), Lb._store_digest()), "load"
    for i in range(3):
        cr, cc, cv = _bench_candidates(wl, i)
        monkeypatch.setenv(knob, "1")
        sa = La.synapto_step(0.01, cr, cc, cv)
        monkeypatch.setenv(knob, "0")
        sb = Lb.synapto_step(0.01, cr, cc, cv)
        assert sa == sb, i
        assert sa["n_scattered"] > 0, sa
        assert np.array_equal(La._store_digest(), Lb._store_digest()), f"step {i}"
    monkeypatch.delenv(knob)


def _exported(L, n_in, n_out):
    ex = L.export_scattered()
    H = HostLayer(n_in, n_out).load_encoded(ex["row_byte_start"], ex["row_elem_start"], ex["idx"], ex["val"])
    H.set_scales(np.asarray(L.get_value_scales(), np.float32))
    return H


@pytest.fixture(scope="module", params=[(5120, 1310720, 20261206), (32768, 204800, 20261207)],
                ids=["gate", "down"])
def c4_layer(hip, request):
    n_in, n_out, seed = request.param
    L = hip.SparseLinearLayer(n_in, n_out, 1)
    nnz = L.load_synthetic(seed, 0.1, 0.02, 0.95)
    assert abs(nnz / (n_in * n_out) - 0.1) < 0.001
    return L, _exported(L, n_in, n_out), n_in, n_out, seed


@pytest.mark.parametrize("B,sel", [(8, None), (128, (0, 1, 31, 64, 100, 127))], ids=["B8", "B128"])
def test_config4_gate_and_down_shapes(hip, c4_layer, B, sel):
    L, H, n_in, n_out, seed = c4_layer
    x = np.random.default_rng(seed + B).normal(size=(B, n_in)).astype(np.float32)
    y = L.forward_dense(x)
    assert y.shape == (B, n_out) and np.all(np.isfinite(y))
    rows = np.arange(B) if sel is None else np.array(sel)
    xs = np.ascontiguousarray(x[rows])
    assert_close_terms(y[rows], H.forward_dense(xs, threads=T), H.forward_dense(xs, absmode=True, threads=T),
                       f"c4 {n_in}x{n_out} B{B}")


def _rank_layer(hip, rng, rank):
    """Scattered synapses outside a set of block4 tiles, every weight code
    drawn (no NaN code), scales of the given rank."""
    n_in, n_out = 300, 1040
    nbr, nbc = n_in // 4, n_out // 4
    keys = np.sort(rng.choice(nbr * nbc, 300, replace=False))
    br, bc = (keys // nbc).astype(np.int32), (keys % nbc).astype(np.int32)
    codes = rng.integers(0, 16, (len(keys), 16)).astype(np.uint8)
    codes[codes == 8] = 0
    tiles = (codes | np.uint8(1 << 4)).ravel()
    cover = np.zeros((n_in, n_out), bool)
    for r, c in zip(br, bc):
        cover[4 * r:4 * r + 4, 4 * c:4 * c + 4] = True
    mask = (rng.random((n_in, n_out)) < 0.05) & ~cover
    mask[7, :] = ~cover[7, :]  # one long row (several work items)
    mask[11, :] = False  # an empty row
    ptrs = np.concatenate([[0], np.cumsum(mask.sum(1))]).astype(np.int32)
    cols = np.nonzero(mask)[1].astype(np.int32)
    q = rng.normal(0, 2, len(cols)).astype(np.float32)
    L = hip.SparseLinearLayer(n_in, n_out, len(cols) + 16 * len(keys) + 64)
    L.load_weights(ptrs, cols, q)
    L.load_block4_tiles(br, bc, tiles)
    L.set_scale_rank(rank)
    vs = rng.uniform(-1.5, 1.5, n_in * rank).astype(np.float32)
    os_ = rng.uniform(-1.5, 1.5, n_out * rank).astype(np.float32)
    L.set_value_scales(vs)
    L.set_output_scales(os_)
    # the decoded codes at unit scale (the oracle's dense view), times S
    D = (HostLayer(n_in, n_out).load_csr(ptrs, cols, w=q).load_tiles(br, bc, tiles).dense()
         .astype(np.float64))
    S = vs.reshape(n_in, rank).astype(np.float64) @ os_.reshape(n_out, rank).astype(np.float64).T
    # the device weight is fl32(dec * S): S rounded to fp32 first
    W = D * S.astype(np.float32).astype(np.float64)
    # the sparse-input forward and the sparse-gradient dx read component 0
    # only (sisldo_ops.hpp:302-306,518-529,689-698)
    W0 = D * np.outer(vs[::rank], os_[::rank]).astype(np.float32).astype(np.float64)
    H = (HostLayer(n_in, n_out, rank).load_csr(ptrs, cols, w=q).load_tiles(br, bc, tiles).set_scales(vs, os_))
    return L, W, W0, H, (ptrs, cols, br, bc)


@pytest.mark.parametrize("rank", [3, 4])
def test_scale_ranks_3_and_4(hip, rank, monkeypatch):
    rng = np.random.default_rng(300 + rank)
    L, W, W0, H, (ptrs, cols, br, bc) = _rank_layer(hip, rng, rank)
    n_in, n_out = W.shape
    assert L.get_scale_rank() == rank
    assert not np.allclose(W, W0)  # the extra components matter
    for B in (1, 2, 8, 16, 64, 128):
        x = rng.normal(size=(B, n_in)).astype(np.float32)
        X = x.astype(np.float64)
        assert_close_terms(L.forward_dense(x), X @ W, np.abs(X) @ np.abs(W), f"rank {rank} fwd B{B}")
        g = rng.normal(size=(B, n_out)).astype(np.float32)
        G = g.astype(np.float64)
        dx = L.backward_dense(g, 0.0)
        assert_close_terms(dx, G @ W.T, np.abs(G) @ np.abs(W.T), f"rank {rank} dx B{B}")
        # grad-W does not depend on the scales: (X^T G) at the stored positions
        gs, gb = L.sampled_gradw(x, g)
        XG = X.T @ G
        aXG = np.abs(X).T @ np.abs(G)
        rows = np.repeat(np.arange(n_in), np.diff(ptrs))
        assert_close_terms(gs, XG[rows, cols], aXG[rows, cols], f"rank {rank} gw scattered B{B}")
        slot = np.arange(16)
        tr = (br[:, None] * 4 + slot % 4).ravel()
        tc = (bc[:, None] * 4 + slot // 4).ravel()
        assert_close_terms(gb, XG[tr, tc], aXG[tr, tc], f"rank {rank} gw block4 B{B}")
    # the sparse-input forward, pushed and gathered
    B = 6
    x = rng.normal(size=(B, n_in)).astype(np.float32)
    x[rng.random(x.shape) < 0.8] = 0.0
    x[2, :] = 0.0  # an empty batch row
    xp = np.concatenate([[0], np.cumsum((x != 0).sum(1))]).astype(np.int32)
    xi = np.nonzero(x)[1].astype(np.int32)
    xv = x[x != 0].astype(np.float32)
    X = x.astype(np.float64)
    for push in ("2", "0"):
        monkeypatch.setenv("SILI_PUSH", push)
        y = L.forward_sparse(xp, xi, xv, B)
        assert_close_terms(y, X @ W0, np.abs(X) @ np.abs(W0), f"rank {rank} sparse fwd, SILI_PUSH={push}")
        assert_close_terms(y, H.forward_sparse(xp, xi, xv, B), H.forward_sparse(xp, xi, xv, B, absmode=True),
                           f"rank {rank} sparse fwd vs oracle, SILI_PUSH={push}")
    monkeypatch.delenv("SILI_PUSH")
    # the sparse-gradient backward at lr 0
    g = rng.normal(size=(B, n_out)).astype(np.float32)
    g[rng.random(g.shape) < 0.7] = 0.0
    gp = np.concatenate([[0], np.cumsum((g != 0).sum(1))]).astype(np.int32)
    gi = np.nonzero(g)[1].astype(np.int32)
    gv = g[g != 0].astype(np.float32)
    G = g.astype(np.float64)
    dx = L.backward_sparse(x, gp, gi, gv, B, 0.0)
    assert_close_terms(dx, G @ W0.T, np.abs(G) @ np.abs(W0.T), f"rank {rank} sparse dx")
    assert_close_terms(dx, H.backward_sparse(x, gp, gi, gv, B)[0],
                       H.backward_sparse(x, gp, gi, gv, B, absmode=True)[0], f"rank {rank} sparse dx vs oracle")
