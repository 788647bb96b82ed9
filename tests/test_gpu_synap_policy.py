"""GPU: the reference's synaptogenesis policy (build_probes, synap_row_step /
synap_step) on the device store against the oracle's restatement (pinned to
the compiled reference in test_synap_policy_oracle.py): probes, structure
byte for byte (scattered and block4), out_degree and the cursor after every
call, over random sequences with promotion and demotion; then an update with
trainable output scales reads the policy's out_degree."""
import numpy as np
import pytest

from oracle import HostLayer
from test_synap_policy_oracle import accum, policy_case

pytestmark = pytest.mark.gpu


def gpu_policy_layer(hip, c, cls="SparseLinearLayerDeterministic"):
    L = getattr(hip, cls)(c["n_in"], c["n_out"], 9 * len(c["cols"]) + 16 * len(c["br"]) + 4096)
    L.load_weights_with_importance(c["ptrs"], c["cols"], c["w"], c["imp"])
    L.load_block4_tiles(c["br"], c["bc"], c["tiles"])
    # rows reserve what the pinned reference layers reserve (blank_fraction 8)
    L.expand_headroom(8.0)
    return L


def host_policy_layer(c):
    H = HostLayer(c["n_in"], c["n_out"]).load_csr(c["ptrs"], c["cols"], w=c["w"], imp=c["imp"])
    H.load_tiles(c["br"], c["bc"], c["tiles"])
    H.out_deg = np.bincount(c["cols"], minlength=c["n_out"]).astype(np.int32)
    return H


def assert_same(L, H, what):
    e = L.export_scattered()
    assert np.array_equal(e["row_elem_start"], H.row_elem_start), what + ": elem_start"
    assert np.array_equal(e["row_byte_start"], H.row_byte_start), what + ": byte_start"
    assert np.array_equal(e["idx"], H.idx[:len(e["idx"])]) and np.array_equal(e["val"], H.val[:len(e["val"])]), \
        what + ": bytes"
    b = L.export_block4()
    assert np.array_equal(b["br"], H.tile_br) and np.array_equal(b["bc"], H.tile_bc), what + ": tiles"
    assert np.array_equal(b["tiles"], H.tiles[:16 * len(b["br"])]), what + ": tile bytes"
    assert np.array_equal(L.out_degree, H.out_deg), what + ": out_degree"


def feed_accumulators(L, rng, n_in, n_out):
    """Accumulators with ties: one forward/backward at batch 1 with inputs and
    gradients of k * 0.5 (exact sums), from zero."""
    L.zero_accum()
    x = accum(rng, n_in)[None, :]
    dy = accum(rng, n_out)[None, :]
    L.forward_dense(x)
    L.backward_dense(dy, 0.0)
    return L.neuron_input_accum.copy(), L.neuron_grad_accum.copy()


@pytest.mark.parametrize("seed", range(4))
def test_synap_policy_matches_oracle(hip, seed):
    c = policy_case(seed)
    L, H = gpu_policy_layer(hip, c), host_policy_layer(c)
    rng = c["rng"]
    assert_same(L, H, "load")
    for it in range(36):
        what = f"seed {seed} call {it}"
        if it % 3 == 0:
            k = int(rng.integers(0, 7))
            per_row = bool(rng.integers(0, 2))
            ai, ag = feed_accumulators(L, rng, c["n_in"], c["n_out"])
            np.testing.assert_array_equal(ai, np.abs(ai))
            L.build_probes(k, per_row)
            H.build_probes(ai, ag, k, per_row)
            pr, pc, pv = L.get_probes()
            assert np.array_equal(pr, H.probes[0][:H.probe_nnz]) and np.array_equal(pc, H.probes[1][:H.probe_nnz])
            assert np.array_equal(pv, H.probes[2][:H.probe_nnz]), what + ": probes"
        if (it // 12) % 2 == 0:
            cutoff, max_rw = float(rng.choice([0.0, 0.3])), int(rng.integers(10, 30))
        else:
            cutoff, max_rw = float(rng.choice([0.6, 1.2, 2.5])), int(rng.integers(2, 12))
        max_prune = int(rng.integers(1, 9))
        eps = float(rng.choice([1e-3, 0.75]))
        if it % 5 == 4:  # explicit row
            row = int(rng.integers(0, 3 * c["n_in"]))
            assert L.synap_row_step(row, cutoff, max_rw, max_prune, eps) == \
                H.synap_row_step(row, cutoff, max_rw, max_prune, eps)[0], what
        else:
            assert L.synap_step(cutoff, max_rw, max_prune, eps) == H.synap_step(cutoff, max_rw, max_prune, eps), what
        assert_same(L, H, what)
    # forward over the edited structure
    x = rng.normal(size=(3, c["n_in"])).astype(np.float32)
    from util import assert_close_terms
    assert_close_terms(L.forward_dense(x), H.forward_dense(x), H.forward_dense(x, absmode=True), "forward")


def test_probes_follow_accumulators(hip):
    """build_probes keeps the accumulators it staged, and its top-k
    selections over them, while only policy calls and calls that read the
    layer run (exports, info, synchronize); after a call that changes them
    (backward, zero_accum) it reads them again.  Probes match the
    oracle's over the accumulators at each call."""
    c = policy_case(6)
    L, H = gpu_policy_layer(hip, c), host_policy_layer(c)
    rng = np.random.default_rng(11)
    n_in, n_out = c["n_in"], c["n_out"]

    def probes_match(k, per_row, what):
        ai, ag = L.neuron_input_accum.copy(), L.neuron_grad_accum.copy()
        L.build_probes(k, per_row)
        H.build_probes(ai, ag, k, per_row)
        pr, pc, pv = L.get_probes()
        n = H.probe_nnz
        assert np.array_equal(pr, H.probes[0][:n]) and np.array_equal(pc, H.probes[1][:n]) and \
            np.array_equal(pv, H.probes[2][:n]), what
        return ai, ag

    feed_accumulators(L, rng, n_in, n_out)
    a0 = probes_match(4, False, "first")
    for it in range(6):
        assert L.synap_step(0.3, 20, 4, 1e-3) == H.synap_step(0.3, 20, 4, 1e-3)
        L.synchronize()
        L.info()
        assert_same(L, H, f"step {it}")
        probes_match([4, 4, 3, 5, 4, 2][it], it % 2 == 1, f"cached, call {it}")
    L.forward_dense(accum(rng, n_in)[None, :])
    L.backward_dense(accum(rng, n_out)[None, :], 0.0)  # both accumulators change
    a1 = probes_match(4, False, "after backward")
    assert not np.array_equal(a0[0], a1[0]) and not np.array_equal(a0[1], a1[1])
    probes_match(3, True, "after backward, per row")
    L.zero_accum()
    probes_match(4, False, "after zero_accum")
    assert L.get_probes()[2].size == 0 or not L.get_probes()[2].any()


def test_update_after_policy_uses_its_out_degree(hip):
    """The output scales' step divides by out_degree and skips a column whose
    out_degree is 0 (linear_disldo.hpp:2061-2064); the policy's count differs
    from the stored synapses once it has removed a block4 slot (loads count
    scattered synapses only) and demoted the tile."""
    n_in, n_out = 8, 6
    ptrs = np.array([0, 0, 0, 0, 0, 1, 2, 3, 4], np.int32)
    cols = np.array([0, 1, 2, 3], np.int32)  # rows 4-7
    w = np.array([1.0, -1.5, 2.0, 0.5], np.float32)
    imp = np.full(4, 6.0, np.float32)
    tile = np.zeros(16, np.uint8)
    tile[0 * 4 + 0] = 0x03   # row 0, col 0: importance 0
    tile[1 * 4 + 1] = 0x02   # row 1, col 1: importance 0
    c = dict(n_in=n_in, n_out=n_out, ptrs=ptrs, cols=cols, w=w, imp=imp, br=np.array([0], np.int32),
             bc=np.array([0], np.int32), tiles=tile)
    L, H = gpu_policy_layer(hip, c), host_policy_layer(c)
    assert L.synap_row_step(0, 1.0, 10) and H.synap_row_step(0, 1.0, 10)[0]
    assert_same(L, H, "after the demotion")
    assert H.n_tiles == 0 and H.out_deg[0] == 0 and H.out_degree()[0] == 1
    rng = np.random.default_rng(3)
    os_ = rng.uniform(0.5, 1.5, n_out).astype(np.float32)
    L.set_output_scales(os_)
    H.set_scales(None, os_)
    H.output_scale_trainable = True
    for step in range(2):
        x = rng.normal(size=(1, n_in)).astype(np.float32)
        dy = rng.normal(size=(1, n_out)).astype(np.float32)
        L.forward_dense(x)
        L.backward_dense(dy, 0.05)
        H.backward_train(x, dy, 0.05)
        assert np.array_equal(L.export_scattered()["val"], H.val[:H.nnz])
        got = np.array([L.get_output_scale_k(col, 0) for col in range(n_out)], np.float32)
        assert np.array_equal(got, H.output_scale), f"step {step}: output scales"
        assert got[0] == os_[0], "column 0 (out_degree 0) takes no step"


@pytest.mark.parametrize("patch", [True, False])
@pytest.mark.parametrize("case", ["scattered_low", "tile_low", "both_low"])
def test_synapse_stored_twice(hip, monkeypatch, case, patch):
    """A synapse held both in its row and in a live tile slot: the removal
    takes the copy the reference takes, by row patch and by the bulk
    pipeline (pinned against the compiled reference in
    test_synap_policy_oracle.py)."""
    monkeypatch.setenv("SILI_POLICY_PATCH", "1" if patch else "0")
    n_in, n_out = 4, 12
    ptrs = np.array([0, 0, 3, 3, 3], np.int32)
    cols = np.array([2, 5, 9], np.int32)
    w = np.array([1.0, -1.5, 2.0], np.float32)
    imp_s, imp_code = {"scattered_low": (0.0, 7), "tile_low": (6.0, 0), "both_low": (0.0, 1)}[case]
    imp = np.array([6.0, imp_s, 6.0], np.float32)
    tile = np.zeros(16, np.uint8)
    tile[1 * 4 + 1] = (imp_code << 4) | 0x3
    tile[2 * 4 + 1] = 0x72
    tile[3 * 4 + 0] = 0x71
    c = dict(n_in=n_in, n_out=n_out, ptrs=ptrs, cols=cols, w=w, imp=imp, br=np.array([0], np.int32),
             bc=np.array([1], np.int32), tiles=tile)
    L, H = gpu_policy_layer(hip, c), host_policy_layer(c)
    assert_same(L, H, "load")
    assert L.synap_row_step(1, 1.0, 30, 8, 1e-3) == H.synap_row_step(1, 1.0, 30, 8, 1e-3)[0]
    assert_same(L, H, case)
