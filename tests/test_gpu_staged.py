"""GPU: the dense forward at batches 65..128 with the input staged in LDS slice
by slice (csrc/staged.hip) against the oracle (linear_disldo.hpp:68-126) and
against the segment gather (SILI_STAGED=0).  Layers with several input slices
of 256 rows and a partial last one, an output row with more than 64 synapses
in one slice (read in several passes), empty output rows, rank-1 value and
output scales, batches 68..128 (lanes past the batch idle); the slice copy
follows structural edits."""
import numpy as np
import pytest

from oracle import HostLayer
from tests.util import assert_close_terms

pytestmark = pytest.mark.gpu


def staged_case(n_in, n_out, density, seed):
    rng = np.random.default_rng(seed)
    rows = []
    for i in range(n_in):
        c = np.flatnonzero(rng.random(n_out) < density)
        if rng.random() < 0.97:
            c = np.union1d(c, [5])  # output 5: nearly every input (> 64 per slice)
        c = c[(c < 7) | (c > 9)]   # outputs 7..9: no synapse
        rows.append(c)
    ptrs = np.concatenate([[0], np.cumsum([len(c) for c in rows])]).astype(np.int32)
    cols = np.concatenate(rows).astype(np.int32)
    q = rng.normal(0, 0.5, len(cols)).astype(np.float32)
    vs = rng.uniform(0.5, 1.5, n_in).astype(np.float32)
    os_ = rng.uniform(0.5, 1.5, n_out).astype(np.float32)
    return ptrs, cols, q, vs, os_


def make(hip, n_in, n_out, density, seed, scales=True):
    ptrs, cols, q, vs, os_ = staged_case(n_in, n_out, density, seed)
    H = HostLayer(n_in, n_out).load_csr(ptrs, cols, w=q)
    L = hip.SparseLinearLayer(n_in, n_out, 4 * len(cols) + 4096)
    L.load_weights(ptrs, cols, q)
    if scales:
        H.set_scales(vs, os_)
        L.set_value_scales(vs)
        L.set_output_scales(os_)
    return H, L


@pytest.mark.parametrize("B", [68, 100, 128])
@pytest.mark.parametrize("shape", [(700, 1000, 0.1, True), (256, 333, 0.3, False), (1500, 260, 0.05, True)])
def test_staged_forward_matches_oracle(hip, monkeypatch, B, shape):
    n_in, n_out, density, scales = shape
    H, L = make(hip, n_in, n_out, density, n_in + B, scales)
    rng = np.random.default_rng(B)
    x = rng.normal(size=(B, n_in)).astype(np.float32)
    monkeypatch.setenv("SILI_STAGED", "1")
    y = L.forward_dense(x)
    assert_close_terms(y, H.forward_dense(x), H.forward_dense(x, absmode=True), f"staged {shape} B{B}")
    assert np.all(y[:, 7:10] == 0)
    monkeypatch.setenv("SILI_STAGED", "0")
    y0 = L.forward_dense(x)
    assert_close_terms(y, y0, H.forward_dense(x, absmode=True), f"staged vs segments {shape} B{B}")


def test_staged_forward_after_structure_changes(hip, monkeypatch):
    """The slice copy is rebuilt after each synaptogenesis step (regrowth,
    then pruning half): staged and segment gathers agree after each."""
    H, L = make(hip, 700, 1000, 0.1, 3)
    rng = np.random.default_rng(4)
    x = rng.normal(size=(128, 700)).astype(np.float32)

    def agree(what):
        monkeypatch.setenv("SILI_STAGED", "1")
        a = L.forward_dense(x)
        monkeypatch.setenv("SILI_STAGED", "0")
        b = L.forward_dense(x)
        np.testing.assert_allclose(a, b, rtol=1e-5, atol=1e-5, err_msg=what)

    agree("loaded")
    e = np.zeros(0, np.int32)
    cr = rng.integers(0, 700, 2000).astype(np.int32)
    cc = rng.integers(0, 1000, 2000).astype(np.int32)
    L.synapto_step(0.2, cr, cc, rng.normal(0, 0.3, 2000).astype(np.float32))
    agree("after a synaptogenesis step")
    L.synapto_step(0.5, e, e, np.zeros(0, np.float32))
    agree("after pruning half")


def test_wide_sparse_layer_stays_on_segment_gather(hip):
    """Fewer synapses than (row, slice) pairs: no slice copy, the segment
    gather runs, and the result matches the oracle."""
    from tests.test_gpu_stream import kernel_counts
    n_in, n_out = 20000, 40
    rng = np.random.default_rng(11)
    keep = rng.random((n_in, n_out)) < 0.0005  # ~400 synapses; 40 rows x 80 slices
    ptrs = np.concatenate([[0], np.cumsum(keep.sum(1))]).astype(np.int32)
    cols = np.nonzero(keep)[1].astype(np.int32)
    q = rng.normal(0, 0.5, len(cols)).astype(np.float32)
    H = HostLayer(n_in, n_out).load_csr(ptrs, cols, w=q)
    L = hip.SparseLinearLayer(n_in, n_out, len(cols) + 64)
    L.load_weights(ptrs, cols, q)
    x = rng.normal(size=(128, n_in)).astype(np.float32)
    counts = kernel_counts(hip, L, lambda: assert_close_terms(
        L.forward_dense(x), H.forward_dense(x), H.forward_dense(x, absmode=True), "wide sparse B128"))
    assert "fwd:gather_staged" not in counts and "fwd:slices" not in counts, counts
