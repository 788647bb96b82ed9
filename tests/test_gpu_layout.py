"""GPU: the reference's scattered-store reservations on the device layer
(export_layout) against their restatement (oracle.ScatteredReservations,
pinned to the compiled reference in tests/test_layout_oracle.py), the budget
refusals, synap_step running out of room with the reference's message and
state, compact's re-encoding of code 8, and the state_dict round trip of
sili/sparse_rnn.py:817-853."""
import numpy as np
import pytest

from oracle import HostLayer, ScatteredReservations, row_content
from test_layout_oracle import random_csr
from util import assert_close_terms

pytestmark = pytest.mark.gpu


def content(L):
    e = L.export_scattered()
    return row_content(e["row_byte_start"], e["row_elem_start"])


def check(L, S, what):
    rb, re_ = content(L)
    got, want = L.export_layout(), S.layout(rb, re_)
    for k in ("byte_start", "byte_end", "elem_start", "elem_end"):
        assert np.array_equal(got[k], want[k]), f"{what}: {k}"
    return rb, re_


@pytest.mark.parametrize("seed", range(4))
def test_reservations_match_restatement(hip, seed):
    rng = np.random.default_rng(300 + seed)
    n_in, n_out = int(rng.integers(5, 40)), int(rng.choice([37, 300, 20000]))
    ptrs, idx, w = random_csr(rng, n_in, n_out, float(rng.uniform(1, 12)))
    mw = 4 * len(idx) + 64 * n_in
    L = hip.SparseLinearLayer(n_in, n_out, mw)
    S = ScatteredReservations(n_in, mw)
    check(L, S, "construction")
    L.load_weights(ptrs, idx, w)
    rb, re_ = content(L)
    S.load(rb, re_)
    check(L, S, "load")
    for step, (op, arg) in enumerate([("compact", None), ("expand", 0.5), ("expand", 0.0), ("expand_to", (7, 0.3)),
                                      ("equalize", (9, 0)), ("equalize", (12, 40)), ("compact", None),
                                      ("expand", 0.2)]):
        if op == "compact":
            L.compact()
            S.compact(rb, re_)
        elif op == "expand":
            L.expand_headroom(arg)
            S.expand(rb, re_, arg)
        elif op == "expand_to":
            L.expand_headroom_to(*arg)
            S.expand(rb, re_, arg[1], arg[0])
        else:
            L.equalize_to_capacity(*arg)
            S.equalize_to_capacity(*arg)
        rb, re_ = check(L, S, f"step {step} {op}{arg}")
        if op == "equalize":
            for k in range(n_in + 3):
                L.equalizer_step()
                S.equalizer_step()
                rb, re_ = check(L, S, f"step {step} equalizer {k}")
    # the layer computes as before: reservations do not touch the synapses
    H = HostLayer(n_in, n_out).load_csr(ptrs, idx, w=w)
    x = rng.normal(size=(3, n_in)).astype(np.float32)
    np.testing.assert_allclose(L.forward_dense(x), H.forward_dense(x), rtol=1e-5, atol=1e-5)


def test_budget_refusals(hip):
    rng = np.random.default_rng(7)
    n_in, n_out = 24, 500
    ptrs, idx, w = random_csr(rng, n_in, n_out, 10.0)
    nnz = len(idx)
    L, S = hip.SparseLinearLayer(n_in, n_out, nnz), ScatteredReservations(n_in, nnz)
    L.load_weights(ptrs, idx, w)
    rb, re_ = content(L)
    S.load(rb, re_)
    for f in (0.2, 0.01):
        with pytest.raises(MemoryError):
            L.expand_headroom(f)
        check(L, S, f"after a refused expand {f}")
    with pytest.raises(MemoryError):
        L.expand_headroom_to(1000)
    with pytest.raises(MemoryError):
        L.expand_headroom_to(-1)
    small, Ss = hip.SparseLinearLayer(n_in, n_out, 5), ScatteredReservations(n_in, 5)
    small.load_weights(ptrs, idx, w)
    Ss.load(rb, re_)
    check(small, Ss, "load beyond max_weights")
    L2, S2 = hip.SparseLinearLayer(n_in, n_out, 3 * nnz), ScatteredReservations(n_in, 3 * nnz)
    L2.load_weights(ptrs, idx, w)
    S2.load(rb, re_)
    with pytest.raises(MemoryError):
        L2.equalize_to_capacity(4 * nnz // n_in)
    with pytest.raises(MemoryError):
        S2.equalize_to_capacity(4 * nnz // n_in)
    check(L2, S2, "after a refused equalize_to_capacity")


@pytest.mark.parametrize("seed", range(6))
def test_policy_runs_out_of_room(hip, seed):
    from test_gpu_synap_policy import assert_same
    from test_synap_policy_oracle import accum, policy_case
    c = policy_case(seed, n_in=24, n_out=400, density=0.03, tile_density=0.03)
    blank = [0.0, 0.1, 0.0, 0.15, 0.0, 0.05][seed]
    L = hip.SparseLinearLayerDeterministic(c["n_in"], c["n_out"], 4 * len(c["cols"]) + 16 * len(c["br"]) + 4096)
    L.load_weights_with_importance(c["ptrs"], c["cols"], c["w"], c["imp"])
    L.load_block4_tiles(c["br"], c["bc"], c["tiles"])
    L.expand_headroom(blank)
    H = HostLayer(c["n_in"], c["n_out"]).load_csr(c["ptrs"], c["cols"], w=c["w"], imp=c["imp"])
    H.load_tiles(c["br"], c["bc"], c["tiles"])
    H.out_deg = np.bincount(c["cols"], minlength=c["n_out"]).astype(np.int32)
    rb, re_ = content(L)
    S = ScatteredReservations(c["n_in"], 1 << 30).from_absolute(rb, re_, blank)
    check(L, S, "load")
    rng = c["rng"]
    raised = 0
    for it in range(120):
        what = f"seed {seed} call {it}"
        if it % 3 == 0:
            ai, ag = accum(rng, c["n_in"]) + 1.0, accum(rng, c["n_out"]) + 1.0
            k = int(rng.integers(2, 9))
            # the device's accumulators hold ai / ag exactly: a forward and a
            # backward at batch 1 from zero
            L.zero_accum()
            L.forward_dense(ai[None, :])
            L.backward_dense(ag[None, :], 0.0)
            assert np.array_equal(L.neuron_input_accum, ai) and np.array_equal(L.neuron_grad_accum, ag)
            L.build_probes(k)
            H.build_probes(ai, ag, k)
        cutoff = float(rng.choice([0.0, 0.0, 0.3, 1.2]))
        max_rw, max_prune = int(rng.integers(4, 40)), int(rng.integers(0, 3))
        err_h = err_l = None
        try:
            did_h = H.synap_step(cutoff, max_rw, max_prune, 1e-3, reservations=S)
        except RuntimeError as e:
            err_h = str(e)
        try:
            did_l = L.synap_step(cutoff, max_rw, max_prune, 1e-3)
        except RuntimeError as e:
            err_l = str(e)
        assert err_l == err_h, what + ": error"
        if err_h is None:
            assert did_l == did_h, what + ": return"
        else:
            raised += 1
        assert_same(L, H, what)
        check(L, S, what)
    assert raised > 0, "no row ran out of room"


def test_compact_reencodes_code8(hip):
    n_in, n_out = 6, 10
    ptrs = np.array([0, 2, 3, 3, 5, 6, 8], np.int32)
    cols = np.array([1, 7, 4, 0, 9, 3, 2, 8], np.int32)
    byts = np.array([0x83, 0x38, 0x88, 0x12, 0x8F, 0xF8, 0x21, 0x80], np.uint8)  # (w << 4) | imp
    L = hip.SparseLinearLayer(n_in, n_out, 64)
    L.load_weight_bytes(ptrs, cols, byts)
    assert np.array_equal(L.export_scattered()["val"], byts)
    x = np.ones((1, n_in), np.float32)
    assert np.isnan(L.forward_dense(x)).any()  # code 8 decodes to NaN
    L.compact()
    want = np.array([0x03, 0x30, 0x00, 0x12, 0x0F, 0xF0, 0x21, 0x00], np.uint8)
    assert np.array_equal(L.export_scattered()["val"], want)
    H = HostLayer(n_in, n_out).load_csr(ptrs, cols, bytes_=want)
    np.testing.assert_allclose(L.forward_dense(x), H.forward_dense(x), rtol=1e-6)


def state_dict(layer):
    """_sparse_linear_layer_state_dict (sili/sparse_rnn.py:817-838)."""
    n = layer.n_inputs
    return {"ptrs": np.array(layer.ptrs), "indices": np.array(layer.indices),
            "weights": np.array(layer.weights_vals), "importance": np.array(layer.importance),
            "value_scale": np.array([layer.get_value_scale(r) for r in range(n)], dtype=np.float32),
            "importance_scale": np.array([layer.get_importance_scale(r) for r in range(n)], dtype=np.float32)}


def load_state_dict(layer, d):
    """_sparse_linear_layer_load_state_dict (sili/sparse_rnn.py:841-853)."""
    layer.load_weights(np.asarray(d["ptrs"], dtype=np.int32), np.asarray(d["indices"], dtype=np.int32),
                       np.asarray(d["weights"], dtype=np.float32))
    for r in range(layer.n_inputs):
        layer.set_value_scale_raw(r, float(d["value_scale"][r]))
        layer.set_importance_scale_raw(r, float(d["importance_scale"][r]))


def test_state_dict_round_trip(hip):
    from train_util import add_tiles, make_train_case
    c = add_tiles(make_train_case(40, 37, 0.1, 51), seed=51)
    L = hip.SparseLinearLayer(40, 37, 40 * 37)
    L.load_weights_with_importance(c["ptrs"], c["cols"], c["w"], c["imp"])
    L.load_block4_tiles(c["br"], c["bc"], c["tiles"])
    L.set_value_scales(c["vs"])
    for r in range(0, 40, 3):
        L.set_importance_scale_raw(r, 0.5 + r)
    H = HostLayer(40, 37).load_csr(c["ptrs"], c["cols"], w=c["w"], imp=c["imp"])
    H.load_tiles(c["br"], c["bc"], c["tiles"])
    # the saved arrays are the reference's combined absolute CSR
    # (delta_csr_combined_to_absolute): scattered and tile synapses merged
    d = state_dict(L)
    hp, hi, hw, himp = H.absolute()
    assert np.array_equal(d["ptrs"], hp) and np.array_equal(d["indices"], hi)
    assert np.array_equal(d["weights"], hw) and np.array_equal(d["importance"], himp)
    assert np.array_equal(d["value_scale"], np.asarray(c["vs"], np.float32))
    # reload onto a fresh layer: every synapse scattered, same true weights
    L2 = hip.SparseLinearLayer(40, 37, 40 * 37)
    load_state_dict(L2, d)
    d2 = state_dict(L2)
    for k in ("ptrs", "indices", "weights", "value_scale", "importance_scale"):
        assert np.array_equal(d2[k], d[k]), k
    assert not np.any(d2["importance"])  # importance is not restorable (load_weights has no path for it)
    x = np.random.default_rng(3).normal(size=(4, 40)).astype(np.float32)
    H.set_scales(np.asarray(c["vs"], np.float32))
    assert_close_terms(L2.forward_dense(x), L.forward_dense(x), H.forward_dense(x, absmode=True), "reloaded fwd")
