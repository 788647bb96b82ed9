"""CPU: the reference's scattered-store reservations (DeltaCSRLayout with
blank space between rows) and the room checks of its in-place edits, against
the restatement the device is checked with (oracle.ScatteredReservations and
the oracle's synap_row_step with reservations), both driven side by side with
the compiled reference (SparseLinearLayer's budgets restated around the
reference's own from_absolute / compact / expand_headroom[_to] /
delta_csr_shift_row / delta_csr_equalize_step, ref_shim.cpp):

- loads, compact, expand_headroom[_to] at several blank fractions,
  equalize_to_capacity (default and explicit bytes), equalizer_step sweeps;
- budget refusals (MemoryError) of expand_headroom[_to] and of the shifts,
  with the state they leave;
- synap_row_step sequences on rows with little room: the RuntimeError, its
  message, and the state left behind (removals and earlier inserts applied).
"""
import numpy as np
import pytest

from oracle import HostLayer, RefLayer, ScatteredReservations, have_ref, row_content

pytestmark = pytest.mark.skipif(not have_ref(), reason="reference build (oracle/_ref) absent")


def random_csr(rng, n_in, n_out, mean):
    lens = rng.poisson(mean, n_in)
    lens[rng.random(n_in) < 0.15] = 0  # empty rows
    lens = np.minimum(lens, n_out)
    cols = [np.sort(rng.choice(n_out, size=int(k), replace=False)) for k in lens]
    ptrs = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    idx = np.concatenate(cols).astype(np.int32) if len(cols) else np.zeros(0, np.int32)
    w = rng.normal(0, 2, len(idx)).astype(np.float32)
    return ptrs, idx, w


def check(R, S, what):
    bs, es, _, _ = R.export()
    rb, re_ = row_content(bs, es)
    got, want = R.layout(), S.layout(rb, re_)
    for k in ("byte_start", "byte_end", "elem_start", "elem_end"):
        assert np.array_equal(got[k], want[k]), f"{what}: {k}"
    return rb, re_


@pytest.mark.parametrize("seed", range(4))
def test_reservations_follow_reference(seed):
    rng = np.random.default_rng(300 + seed)
    n_in, n_out = int(rng.integers(5, 40)), int(rng.choice([37, 300, 20000]))
    ptrs, idx, w = random_csr(rng, n_in, n_out, float(rng.uniform(1, 12)))
    mw = 4 * len(idx) + 64 * n_in
    R = RefLayer.sll(n_in, n_out, mw)
    S = ScatteredReservations(n_in, mw)
    rb, re_ = check(R, S, "construction")
    R.load_weights(ptrs, idx, w)
    rb, re_ = row_content(*R.export()[:2])
    S.load(rb, re_)
    check(R, S, "load")
    for step, (op, arg) in enumerate([("compact", None), ("expand", 0.5), ("expand", 0.0), ("expand_to", (7, 0.3)),
                                      ("equalize", (9, 0)), ("equalize", (12, 40)), ("compact", None),
                                      ("expand", 0.2)]):
        if op == "compact":
            R.compact_layer()
            S.compact(rb, re_)
        elif op == "expand":
            R.expand_headroom(arg)
            S.expand(rb, re_, arg)
        elif op == "expand_to":
            R.expand_headroom_to(*arg)
            S.expand(rb, re_, arg[1], arg[0])
        else:
            R.equalize_to_capacity(*arg)
            S.equalize_to_capacity(*arg)
        rb, re_ = check(R, S, f"step {step} {op}{arg}")
        if op == "equalize":
            for k in range(n_in + 3):  # a full equalizer sweep and then some
                R.equalizer_step()
                S.equalizer_step()
                rb, re_ = check(R, S, f"step {step} equalizer {k}")


def test_budget_refusals_and_what_they_leave():
    rng = np.random.default_rng(7)
    n_in, n_out = 24, 500
    ptrs, idx, w = random_csr(rng, n_in, n_out, 10.0)
    nnz = len(idx)
    # a budget the load fills exactly: every expand asks for more
    R, S = RefLayer.sll(n_in, n_out, nnz), ScatteredReservations(n_in, nnz)
    R.load_weights(ptrs, idx, w)
    rb, re_ = row_content(*R.export()[:2])
    S.load(rb, re_)
    for f in (0.2, 0.01):
        with pytest.raises(MemoryError):
            R.expand_headroom(f)
        with pytest.raises(MemoryError):
            S.expand(rb, re_, f)
        check(R, S, f"after a refused expand {f}")
    with pytest.raises(MemoryError):
        R.expand_headroom_to(1000)
    with pytest.raises(MemoryError):
        S.expand(rb, re_, 0.2, 1000)
    # a load beyond max_weights grows the budgets to fit it
    small = RefLayer.sll(n_in, n_out, 5)
    Ss = ScatteredReservations(n_in, 5)
    small.load_weights(ptrs, idx, w)
    Ss.load(rb, re_)
    check(small, Ss, "load beyond max_weights")
    # equalize_to_capacity past the budget: the rows before the refusing one grow
    R2, S2 = RefLayer.sll(n_in, n_out, 3 * nnz), ScatteredReservations(n_in, 3 * nnz)
    R2.load_weights(ptrs, idx, w)
    S2.load(rb, re_)
    with pytest.raises(MemoryError):
        R2.equalize_to_capacity(4 * nnz // n_in)
    with pytest.raises(MemoryError):
        S2.equalize_to_capacity(4 * nnz // n_in)
    check(R2, S2, "after a refused equalize_to_capacity")
    assert int(S2.e[0]) == 4 * nnz // n_in, "the first rows grew before the refusal"


def _layers(c, blank):
    H = HostLayer(c["n_in"], c["n_out"]).load_csr(c["ptrs"], c["cols"], w=c["w"], imp=c["imp"])
    H.load_tiles(c["br"], c["bc"], c["tiles"])
    R = RefLayer(c["n_in"], c["n_out"], c["ptrs"], c["cols"], c["w"], c["imp"], blank_fraction=blank)
    for t in range(len(c["br"])):
        R.put_tile(int(c["br"][t]), int(c["bc"][t]), c["tiles"][16 * t:16 * t + 16])
    bs, es, _, _ = R.export()
    S = ScatteredReservations(c["n_in"], 1 << 30).from_absolute(*row_content(bs, es), blank)
    return H, R, S


@pytest.mark.parametrize("seed", range(6))
def test_policy_runs_out_of_room_as_the_reference(seed):
    from test_synap_policy_oracle import accum, assert_same, policy_case
    # wide rows (multi-byte deltas), sparse windows: inserts stay scattered
    # instead of being promoted into tiles, so the rows fill up
    c = policy_case(seed, n_in=24, n_out=400, density=0.03, tile_density=0.03)
    H, R, S = _layers(c, [0.0, 0.1, 0.0, 0.15, 0.0, 0.05][seed])
    H.out_deg = R.out_degree().copy()
    rng = c["rng"]
    cur = 0
    raised = inserted = 0
    for it in range(120):
        what = f"seed {seed} call {it}"
        if it % 3 == 0:
            ai, ag = accum(rng, c["n_in"]) + 1.0, accum(rng, c["n_out"]) + 1.0
            k = int(rng.integers(2, 9))
            H.build_probes(ai, ag, k)
            R.build_probes(ai, ag, k)
        cutoff = float(rng.choice([0.0, 0.0, 0.3, 1.2]))
        max_rw, max_prune = int(rng.integers(4, 40)), int(rng.integers(0, 3))
        err_h = err_r = None
        n0 = H.nnz + int(np.count_nonzero(H.tiles[:16 * H.n_tiles]))
        try:
            did_h = H.synap_step(cutoff, max_rw, max_prune, 1e-3, reservations=S)
        except RuntimeError as e:
            err_h = str(e)
        try:
            did_r, nxt = R.synap_row_step(cur, cutoff, max_rw, max_prune, 1e-3)
        except RuntimeError as e:
            err_r = str(e)
        assert err_h == err_r, what + ": error"
        if err_r is not None:
            raised += 1
            if err_r.startswith("block4_demote_tile"):
                break  # the reference leaves that tile half demoted: the states part here
            H.synap_cursor = cur  # the cursor stays where it was (the call threw)
        else:
            assert did_h == did_r, what + ": return"
            cur = nxt
        assert_same(H, R, what)
        check(R, S, what)
        inserted += H.nnz + int(np.count_nonzero(H.tiles[:16 * H.n_tiles])) > n0
    assert raised > 0, "no row ran out of room"
    assert inserted > 0, "no call grew a row"
