"""GPU: the block4 store's reservations (the reference's Block4Store
per-block-row index bytes, tile slots and tile bytes, block4.hpp:1016-1031)
and the optimizer updates' write-back with eviction (merge_row_workspace,
block4.hpp:1367-1462) on the device against the oracle's restatement
(oracle.Block4Reservations, the oracle's updates and policy step, pinned to
the compiled reference in test_block4_reservations_oracle.py and
test_train_oracle.py):

- load_dense_codes (delta_csr_memory.hpp:841-945), then expand_block4_headroom
  / compact_block4 / equalizer_step sequences, refusals at the budget;
- load_block4_tiles reserving as its tiles placed one by one would, refused
  where the budget would refuse or drop;
- the dense and the sparse-gradient update on load_dense_codes layers, with
  the headroom load_dense_codes leaves and after compact_block4: tile bytes,
  tile_is_sparse, the write-back counters and Block4View exact;
- the reference policy's promotions under a small budget (rows grown,
  commits dropped, MemoryError) with the reservations kept exactly.
"""
import numpy as np
import pytest

from oracle import Block4Reservations, HostLayer, ScatteredReservations, block4_put_layer, block4_row_use, row_content
from train_util import check_b4_reservations, dx_bound, dx_bound_tiles, sparse_dy
from util import assert_close_terms

pytestmark = pytest.mark.gpu

SEED = 123  # the update rounding's seed (seed_stochastic_rounding)


def codes(rng, n_in, n_out, density, imp_density):
    wc = np.where(rng.random(n_in * n_out) < density, rng.integers(1, 16, n_in * n_out), 0).astype(np.uint8)
    wc[wc == 8] = 3
    ic = np.where(rng.random(n_in * n_out) < imp_density, rng.integers(1, 8, n_in * n_out), 0).astype(np.uint8)
    return wc, ic


def grid_tiles(n_in, n_out, wc, ic):
    """The tiles load_dense_codes makes: every (br, bc), slot lj*4+li."""
    brows, bcols = (n_in + 3) // 4, (n_out + 3) // 4
    full = np.zeros((brows * 4, bcols * 4), np.uint8)
    full[:n_in, :n_out] = (wc | (ic << 4)).reshape(n_in, n_out)
    t = full.reshape(brows, 4, bcols, 4).transpose(0, 2, 3, 1).reshape(brows * bcols, 16)
    br, bc = np.divmod(np.arange(brows * bcols), bcols)
    return br.astype(np.int32), bc.astype(np.int32), t.ravel()


def loaded(hip, n_in, n_out, wc, ic, cls="SparseLinearLayerDeterministic"):
    L = getattr(hip, cls)(n_in, n_out, n_in * n_out)
    L.load_dense_codes(wc, ic)
    H = HostLayer(n_in, n_out)
    H.load_tiles(*grid_tiles(n_in, n_out, wc, ic))
    H.b4res = Block4Reservations(n_in, n_in * n_out)
    H.b4res.load_dense(n_in, n_out, wc, ic)
    live = (H.tiles[:16 * H.n_tiles].reshape(-1, 16) != 0).sum(1)
    H.b4_flags = (live <= H.b4res.sp).astype(np.uint8)
    return L, H


def use(H):
    return block4_row_use(H.n_in, H.tile_br, H.tile_bc, H.tiles[:16 * H.n_tiles], H.b4_flags[:H.n_tiles])


@pytest.mark.parametrize("n_in,n_out,density,imp", [(16, 24, 0.05, 0.0), (30, 41, 0.3, 0.1), (13, 200, 0.6, 0.3),
                                                    (64, 64, 0.95, 0.0), (37, 530, 0.02, 0.02)])
def test_load_dense_codes_reservations(hip, n_in, n_out, density, imp):
    rng = np.random.default_rng(n_in * 100 + n_out)
    L, H = loaded(hip, n_in, n_out, *codes(rng, n_in, n_out, density, imp))
    check_b4_reservations(L, H, "load_dense_codes")
    d = L.export_block4_layout()
    ui, ue, ut = use(H)
    assert list(d["ui"]) == ui and list(d["ue"]) == ue and list(d["ut"]) == ut, "use"
    assert (d["idx_budget"], d["tile_budget"]) == (H.b4res.idx_budget, H.b4res.tile_budget), "budgets"
    v = L.block4
    assert v.alloc_bytes == sum(H.b4res.ta) and v.used_bytes == sum(ut)


@pytest.mark.parametrize("seed", range(3))
def test_expand_compact_equalize_sequences(hip, seed):
    rng = np.random.default_rng(seed)
    n_in, n_out = int(rng.integers(9, 60)), int(rng.integers(9, 120))
    L, H = loaded(hip, n_in, n_out, *codes(rng, n_in, n_out, float(rng.uniform(0.01, 0.5)), 0.05))
    M = H.b4res
    u = use(H)
    for step in range(30):
        op = int(rng.integers(0, 4))
        if op == 0:
            calls = (L.compact_block4, lambda: M.compact(u[2]))
        elif op == 1:
            f = float(rng.choice([0.0, 0.1, 0.5, 1.0, 30.0]))
            calls = (lambda: L.expand_block4_headroom(f), lambda: M.expand(u[2], f, 16))
        else:
            calls = (L.equalizer_step, lambda: M.equalize_step(*u))
        errs = []
        for call in calls:
            try:
                call()
                errs.append(None)
            except MemoryError:
                errs.append(MemoryError)
        assert errs[0] == errs[1], (seed, step, op)
        check_b4_reservations(L, H, f"seed {seed} step {step} op {op}")


@pytest.mark.parametrize("max_weights", [16, 40, 64, 200])
def test_load_block4_tiles_reservations_and_budget(hip, max_weights):
    rng = np.random.default_rng(max_weights)
    n_in, n_out = 24, 2400
    n = 12
    keys = np.sort(rng.choice(6 * 600, n, replace=False))
    br, bc = (keys // 600).astype(np.int32), (keys % 600).astype(np.int32)
    tiles = np.zeros((n, 16), np.uint8)
    for t in range(n):
        live = rng.choice(16, int(rng.choice([1, 2, 5, 10, 11, 16])), replace=False)
        tiles[t, live] = rng.integers(1, 256, len(live))
    L = hip.SparseLinearLayer(n_in, n_out, max_weights)
    try:
        T, flags = block4_put_layer(n_in, max_weights, br, bc, tiles)
        refused = T.M.dropped > 0
    except MemoryError:
        refused = True
    if refused:
        with pytest.raises(MemoryError):
            L.load_block4_tiles(br, bc, tiles.ravel())
        assert L.block4.tiles == 0 and L.block4.alloc_bytes == 0
        return
    L.load_block4_tiles(br, bc, tiles.ravel())
    H = HostLayer(n_in, n_out).load_tiles(br, bc, tiles.ravel())
    H.b4res, H.b4_flags = T.M, flags
    check_b4_reservations(L, H, f"max_weights {max_weights}")


def _train(L, H, rng, B, lr, steps, sparse, what):
    """steps updates on both layers; L was seeded (seed_stochastic_rounding)
    with SEED just before: update k draws from splitmix64(SEED ^
    splitmix64(k))."""
    from test_gpu_train import _splitmix64
    n_in, n_out = H.n_in, H.n_out
    for step in range(steps):
        x = rng.normal(size=(B, n_in)).astype(np.float32)
        if sparse:
            dp, di, dv, dense = sparse_dy(rng, B, n_out, density=0.5)
            bound = dx_bound_tiles(H, dense, lr, sparse=True) + 1e-30
            dxg = L.backward_sparse(x, dp, di, dv, B, lr)
            seed = _splitmix64(SEED ^ _splitmix64(step + 1))
            dxh, _, _ = H.backward_sparse_train(x, dp, di, dv, B, lr, draw_mode=1, draw_seed=seed)
        else:
            dy = rng.normal(size=(B, n_out)).astype(np.float32)
            bound = dx_bound(H, dy, lr) + dx_bound_tiles(H, dy, lr)
            L.forward_dense(x)
            dxg = L.backward_dense(dy, lr)
            dxh, _, _ = H.backward_train(x, dy, lr)
        w = f"{what} step {step}"
        ex = L.export_block4()
        assert np.array_equal(ex["tiles"], H.tiles[:16 * H.n_tiles]), w + ": tile bytes"
        check_b4_reservations(L, H, w)
        v = L.block4
        assert (v.alloc_bytes, v.dropped_growth_events, v.row_merge_overflow_events,
                v.row_merge_overflow_bytes_dropped) == (sum(H.b4res.ta), H.b4res.dropped, H.b4_counters[1],
                                                        H.b4_counters[2]), w + ": Block4View"
        assert_close_terms(dxg, dxh, bound, w + ": dx")


@pytest.mark.parametrize("sparse", [False, True], ids=["dense_update", "sparse_update"])
@pytest.mark.parametrize("compact", [False, True], ids=["load_headroom", "compacted"])
def test_updates_evict_as_the_reference(hip, sparse, compact):
    """load_dense_codes of a mostly-zero code matrix (sparse-packed and empty
    tiles that the update makes live), then updates; compacted rows evict
    from the first update on."""
    rng = np.random.default_rng(7 + 2 * sparse + compact)
    n_in, n_out = 36, 52
    L, H = loaded(hip, n_in, n_out, *codes(rng, n_in, n_out, 0.15, 0.1))
    if compact:
        L.compact_block4()
        H.b4res.compact(use(H)[2])
    L.seed_stochastic_rounding(SEED)
    _train(L, H, rng, 3, 0.05, 4, sparse, f"sparse={sparse} compact={compact}")
    assert H.b4_counters[0] > 0, "nothing was evicted"


def test_policy_under_a_small_budget(hip):
    """The reference policy's promotions on a layer with a small block4
    budget: rows grown by get_or_create, commits dropped, MemoryError; the
    reservations, tile_is_sparse and the structure as the oracle's after
    every call (pinned in test_block4_reservations_oracle.py)."""
    from test_gpu_synap_policy import assert_same, feed_accumulators
    from test_synap_policy_oracle import policy_case
    events = 0
    for seed, mw in ((2, 160), (3, 96), (5, 120)):
        c = policy_case(seed, n_in=28, n_out=48, density=0.2, tile_density=0.1)
        n_in, n_out = c["n_in"], c["n_out"]
        # tiles whose content fits the budget when placed one by one (those
        # whose commit the budget drops stay empty), then that placement as
        # load_block4_tiles makes it
        br, bc, tiles, _ = block4_put_layer(n_in, mw, c["br"], c["bc"], c["tiles"])[0].canonical()
        T, flags = block4_put_layer(n_in, mw, br, bc, tiles)
        assert T.M.dropped == 0
        L = hip.SparseLinearLayerDeterministic(n_in, n_out, mw)
        L.load_weights_with_importance(c["ptrs"], c["cols"], c["w"], c["imp"])
        L.load_block4_tiles(br, bc, tiles)
        H = HostLayer(n_in, n_out).load_csr(c["ptrs"], c["cols"], w=c["w"], imp=c["imp"])
        H.load_tiles(br, bc, tiles)
        H.out_deg = np.bincount(c["cols"], minlength=n_out).astype(np.int32)
        H.b4res, H.b4_flags = T.M, (flags if len(flags) else np.zeros(1, np.uint8))
        S = ScatteredReservations(n_in, mw).load(*row_content(H.row_byte_start, H.row_elem_start))
        check_b4_reservations(L, H, f"seed {seed} load")
        rng = c["rng"]
        for it in range(60):
            what = f"seed {seed} call {it}"
            if it % 3 == 0:
                ai, ag = feed_accumulators(L, rng, n_in, n_out)
                k = int(rng.integers(1, 8))
                L.build_probes(k)
                H.build_probes(ai, ag, k)
            grow = (it // 10) % 2 == 0
            cutoff, max_rw = (0.0, int(rng.integers(12, 40))) if grow else (float(rng.choice([0.6, 1.2])), 6)
            errs = []
            for call in (lambda: L.synap_step(cutoff, max_rw, 8, 1e-3),
                         lambda: H.synap_step(cutoff, max_rw, 8, 1e-3, reservations=S)):
                try:
                    errs.append((None, call()))
                except (MemoryError, RuntimeError) as e:
                    errs.append((type(e), None))
            assert errs[0] == errs[1], (what, errs)
            events += errs[0][0] is MemoryError
            assert_same(L, H, what)
            check_b4_reservations(L, H, what)
        events += H.b4res.dropped
    assert events > 0, "the budget never bound"
