"""The restatement of the reference's block4 reservations
(oracle.Block4Reservations) against the reference's own compiled Block4Store
(oracle/_ref): per block row the reserved and used index bytes, tile slots
and tile bytes, the budgets and dropped_growth_events, after

- block4_load_dense (load_dense_codes) of code matrices of every density,
  edge tiles included (delta_csr_memory.hpp:841-945);
- compact_block4 / expand_block4_headroom(f) / Block4Store::equalize_step
  sequences (delta_csr_memory.hpp:767-838, block4.hpp:1208-1220);
- tiles placed one by one through get_or_create and a handle's writes on a
  SparseLinearLayer with its constructor's budgets (block4.hpp:648-771,
  906-946, 1170-1183, 1226-1290): rows grown by ensure_row_headroom, commits
  that outgrow a row's room, commits dropped at the tile budget, and
  MemoryError at the index/tile budget.
"""
import numpy as np
import pytest

from oracle import Block4PutModel, Block4Reservations, RefLayer, block4_row_use, have_ref

pytestmark = pytest.mark.skipif(not have_ref(), reason="oracle/_ref not built (needs the reference tree)")


def ref_state(R):
    (ia, ea, ta, ui, ue, ut), ctr = R.block4_reservations()
    return dict(ia=ia, ea=ea, ta=ta, ui=ui, ue=ue, ut=ut, dropped=ctr[0], idx_budget=ctr[3], tile_budget=ctr[4])


def ref_use(R, n_in):
    br, bc, tiles = R.export_tiles()
    flags, _, _ = R.export_tiles_packed()
    return block4_row_use(n_in, br, bc, tiles, flags[:len(br)])


def assert_same(M, use, R, what):
    st = ref_state(R)
    assert list(use[0]) == st["ui"] and list(use[1]) == st["ue"] and list(use[2]) == st["ut"], what + ": use"
    assert M.ia == st["ia"], what + ": index bytes reserved"
    assert M.ea == st["ea"], what + ": tile slots reserved"
    assert M.ta == st["ta"], what + ": tile bytes reserved"
    assert M.dropped == st["dropped"], what + ": dropped growth events"
    assert (M.idx_budget, M.tile_budget) == (st["idx_budget"], st["tile_budget"]), what + ": budgets"


def codes(rng, n_in, n_out, density, imp_density=0.0):
    wc = np.where(rng.random(n_in * n_out) < density, rng.integers(1, 16, n_in * n_out), 0).astype(np.uint8)
    ic = np.where(rng.random(n_in * n_out) < imp_density, rng.integers(1, 16, n_in * n_out), 0).astype(np.uint8)
    return wc, ic


@pytest.mark.parametrize("n_in,n_out,density,imp", [(8, 8, 0.0, 0.0), (16, 24, 0.05, 0.0), (30, 41, 0.3, 0.1),
                                                    (13, 200, 0.6, 0.3), (64, 64, 0.95, 0.0), (5, 3, 1.0, 1.0),
                                                    (37, 530, 0.02, 0.02)])
def test_load_dense_codes_reservations(n_in, n_out, density, imp):
    rng = np.random.default_rng(n_in * 1000 + n_out)
    wc, ic = codes(rng, n_in, n_out, density, imp)
    R = RefLayer.sll(n_in, n_out, 64)
    R.sll_load_dense_codes(wc, ic)
    M = Block4Reservations(n_in, 64)
    use = M.load_dense(n_in, n_out, wc, ic)
    assert_same(M, use, R, "load_dense_codes")
    assert list(use) == [list(u) for u in ref_use(R, n_in)]


@pytest.mark.parametrize("seed", range(4))
def test_compact_expand_equalize_sequences(seed):
    rng = np.random.default_rng(seed)
    n_in, n_out = int(rng.integers(9, 60)), int(rng.integers(9, 120))
    wc, ic = codes(rng, n_in, n_out, float(rng.uniform(0.01, 0.5)), 0.05)
    R = RefLayer.sll(n_in, n_out, 64)
    R.sll_load_dense_codes(wc, ic)
    M = Block4Reservations(n_in, 64)
    use = M.load_dense(n_in, n_out, wc, ic)
    for step in range(40):
        op = int(rng.integers(0, 4))
        what = f"seed {seed} step {step} op {op}"
        calls = [(lambda: R.block4_expand(0.0, 0), lambda: M.compact(use[2]))]
        if op == 1:
            f = float(rng.choice([0.0, 0.1, 0.2, 0.5, 1.0, 3.0]))
            calls = [(lambda: R.block4_expand(f, 16), lambda: M.expand(use[2], f, 16))]
        elif op > 1:
            calls = [(R.block4_equalize_step, lambda: M.equalize_step(*use))]
        for ref_call, model_call in calls:
            errs = []
            for call in (ref_call, model_call):
                try:
                    call()
                    errs.append(False)
                except MemoryError:
                    errs.append(True)
            assert errs[0] == errs[1], what
        assert_same(M, use, R, what)


def test_expand_beyond_the_tile_budget_raises():
    rng = np.random.default_rng(3)
    n_in, n_out = 20, 40
    wc, ic = codes(rng, n_in, n_out, 0.5)
    R = RefLayer.sll(n_in, n_out, 64)
    R.sll_load_dense_codes(wc, ic)
    M = Block4Reservations(n_in, 64)
    use = M.load_dense(n_in, n_out, wc, ic)
    with pytest.raises(MemoryError):
        R.block4_expand(50.0, 16)
    with pytest.raises(MemoryError):
        M.expand(use[2], 50.0, 16)
    assert_same(M, use, R, "after a refused expand")


@pytest.mark.parametrize("seed,max_weights", [(0, 16), (1, 64), (2, 200), (3, 2000), (4, 40)])
def test_tiles_placed_one_by_one(seed, max_weights):
    rng = np.random.default_rng(50 + seed)
    n_in, n_out = 24, 2400  # block columns up to 600: two-byte deltas
    R = RefLayer.sll(n_in, n_out, max_weights)
    T = Block4PutModel(n_in, max_weights)
    n_err = 0
    for step in range(120):
        br = int(rng.integers(0, T.M.rows))
        bc = int(rng.integers(0, (n_out + 3) // 4)) if rng.random() < 0.7 or not T.rows[br] else \
            int(rng.choice(sorted(T.rows[br])))
        live = int(rng.choice([0, 1, 2, 5, 10, 11, 16]))
        tile = np.zeros(16, np.uint8)
        tile[rng.choice(16, live, replace=False)] = rng.integers(1, 256, live)
        try:
            R.sll_put_tile(br, bc, tile)
            ref_err = None
        except MemoryError as e:
            ref_err = e
        try:
            T.put(br, bc, tile)
            err = None
        except MemoryError as e:
            err = e
        assert (ref_err is None) == (err is None), f"step {step}: {ref_err} vs {err}"
        n_err += err is not None
        assert_same(T.M, T.use(), R, f"seed {seed} step {step}")
    if max_weights <= 64:
        assert n_err > 0 or T.M.dropped > 0, "the budget never bound"


@pytest.mark.parametrize("seed,max_weights", [(0, 4000), (1, 400), (2, 160), (3, 96), (4, 4000), (5, 120)])
def test_policy_sequences_keep_the_reference_reservations(seed, max_weights):
    """build_probes + synap_row_step sequences on a SparseLinearLayer with
    its budgets (delta_csr_memory.hpp:1203-1258): tile slots removed through
    handles, demotions, promotions into new tiles (rows grown by
    get_or_create, MemoryError at the budget) and into existing ones (commits
    grown, dropped at the tile budget, maybe_compress).  Structure,
    tile_is_sparse, every block row's reservations and dropped_growth_events
    against the compiled reference after every call."""
    from oracle import HostLayer, ScatteredReservations, row_content
    from test_synap_policy_oracle import accum, policy_case
    c = policy_case(seed, n_in=28, n_out=48, density=0.2, tile_density=0.1)
    n_in, n_out = c["n_in"], c["n_out"]
    rng = c["rng"]
    R = RefLayer.sll(n_in, n_out, max_weights)
    R.load_weights(c["ptrs"], c["cols"], c["w"], c["imp"])
    H = HostLayer(n_in, n_out).load_csr(c["ptrs"], c["cols"], w=c["w"], imp=c["imp"])
    S = ScatteredReservations(n_in, max_weights).load(*row_content(H.row_byte_start, H.row_elem_start))
    T = Block4PutModel(n_in, max_weights)
    tiles = c["tiles"].reshape(-1, 16)
    for t in range(len(c["br"])):
        R.sll_put_tile(int(c["br"][t]), int(c["bc"][t]), tiles[t])
        T.put(int(c["br"][t]), int(c["bc"][t]), tiles[t])
    kept = [(b, cc) for b, row in enumerate(T.rows) for cc in sorted(row)]
    H.load_tiles(np.array([k[0] for k in kept], np.int32), np.array([k[1] for k in kept], np.int32),
                 np.concatenate([T.rows[b][cc][1] for b, cc in kept]) if kept else np.zeros(0, np.uint8))
    H.b4res = T.M
    H.b4_flags = np.array([T.rows[b][cc][0] for b, cc in kept] or [0], np.uint8)
    H.out_deg = R.out_degree().astype(np.int32)
    cur = 0
    n_mem = 0
    for it in range(80):
        what = f"seed {seed} call {it}"
        if it % 3 == 0:
            k = int(rng.integers(1, 8))
            ai, ag = accum(rng, n_in) + 0.5, accum(rng, n_out) + 0.5
            per_row = bool(rng.integers(0, 2))
            H.build_probes(ai, ag, k, per_row)
            R.build_probes(ai, ag, k, per_row)
        grow = (it // 10) % 2 == 0
        cutoff, max_rw = (0.0, int(rng.integers(12, 40))) if grow else (float(rng.choice([0.6, 1.2])), 6)
        errs = []
        for call in (lambda: R.synap_row_step(cur, cutoff, max_rw, 8, 1e-3),
                     lambda: H.synap_row_step(cur, cutoff, max_rw, 8, 1e-3, reservations=S)):
            try:
                errs.append((None, call()))
            except (MemoryError, RuntimeError) as e:
                errs.append((type(e), None))
        assert errs[0][0] == errs[1][0], (what, errs)
        if errs[0][0] is None:
            assert errs[0][1][0] == errs[1][1][0], what
            cur = errs[0][1][1]
        else:
            n_mem += errs[0][0] is MemoryError
        br, bc, tr = R.export_tiles()
        assert np.array_equal(H.tile_br, br) and np.array_equal(H.tile_bc, bc), what + ": tile set"
        assert np.array_equal(H.tiles[:len(tr)], tr), what + ": tile bytes"
        flags = R.export_tiles_packed()[0][:len(br)]
        assert np.array_equal(H.b4_flags[:len(br)], flags), what + ": tile_is_sparse"
        _, _, idx, val = R.export()
        assert np.array_equal(H.val[:len(val)], val), what + ": scattered bytes"
        st = ref_state(R)
        M = H.b4res
        assert (M.ia, M.ea, M.ta, M.dropped) == (st["ia"], st["ea"], st["ta"], st["dropped"]), what + ": reservations"
    if max_weights <= 120:
        assert n_mem > 0 or H.b4res.dropped > 0, "the budget never bound"
