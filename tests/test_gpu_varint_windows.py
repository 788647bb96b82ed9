"""GPU: multi-byte ULEB128 deltas at every byte offset of the 64-byte decode
windows, in both orientations of the store.

Row r of the designed layer holds `off` one-byte deltas, then one 2- or
3-byte delta, then 70 more one-byte deltas, so its multi-byte varint starts
at index byte `off`.  Offsets sweep every lane of the first windows
(including lanes 60-63, where a varint's continuation flags sit at the top
of the wave's terminator mask) and the 508-byte work-item boundary.  The
canonical store of layer A carries the designed rows (backward / grad-W
gather them); layer B = A transposed carries them in its shadow store (its
forward gathers them).  Every kernel variant keyed on the batch runs, and
batch 1 runs through both the segment and the byte-split kernels."""
import numpy as np
import pytest

from oracle import HostLayer
from sili__new_amd.synth import per_row_quantize
from tests.util import assert_close_terms

BATCHES = [1, 2, 4, 8, 12, 64, 128, 256]


@pytest.fixture(params=["1", "2"], autouse=True)
def stream_mode(request, monkeypatch):
    """Batch 1 through the segment kernels ("1": these stores are below the
    stream kernels' default size) and through the byte-split stream kernels
    ("2")."""
    monkeypatch.setenv("SILI_B1_STREAM", request.param)
    yield request.param


def _designed_rows():
    specs = [(off, 300) for off in list(range(0, 200)) + list(range(440, 530))]  # 2-byte deltas
    specs += [(off, 20000) for off in range(0, 140)]                              # 3-byte deltas
    rows = []
    for off, big in specs:
        head = list(range(off))
        nxt = (head[-1] if head else 0) + big
        rows.append(head + list(range(nxt, nxt + 71)))
    return rows


def _layers():
    rows = _designed_rows()
    n_in = len(rows)
    n_out = max(r[-1] for r in rows) + 1
    ptrs = np.concatenate([[0], np.cumsum([len(r) for r in rows])]).astype(np.int32)
    cols = np.concatenate(rows).astype(np.int32)
    w = np.random.default_rng(11).normal(size=len(cols)).astype(np.float32)
    q, s = per_row_quantize(ptrs, w, n_in)
    # transpose: rows of B = columns of A, entries in ascending A-row order
    row_of = np.repeat(np.arange(n_in), np.diff(ptrs)).astype(np.int32)
    order = np.lexsort((row_of, cols))
    tptrs = np.concatenate([[0], np.cumsum(np.bincount(cols, minlength=n_out))]).astype(np.int32)
    tcols = row_of[order]
    tq, ts = per_row_quantize(tptrs, w[order], n_out)
    return (n_in, n_out, ptrs, cols, q, s), (n_out, n_in, tptrs, tcols, tq, ts)


def _pair(hip, spec):
    n_in, n_out, ptrs, cols, q, s = spec
    H = HostLayer(n_in, n_out)
    H.load_csr(ptrs, cols, w=q)
    H.set_scales(s)
    L = hip.SparseLinearLayer(n_in, n_out, len(cols))
    L.load_weights(ptrs, cols, q)
    L.set_value_scales(s)
    return H, L


def test_designed_rows_encode_as_intended():
    """The sweep really places the multi-byte varint at byte `off` (CPU-side
    check of the design, through the oracle's encoder)."""
    (n_in, n_out, ptrs, cols, q, s), _ = _layers()
    H = HostLayer(n_in, n_out)
    H.load_csr(ptrs, cols, w=q)
    starts = H.row_byte_start.astype(np.int64)
    rows = _designed_rows()
    for r, cs in enumerate(rows):
        seg = H.idx[starts[r]:starts[r + 1]]
        cont = np.nonzero(seg & 0x80)[0]
        big = cs[len(cs) - 71] - (cs[len(cs) - 72] if len(cs) > 71 else 0)
        nbytes = 2 if big < 16384 else 3
        off = len(cs) - 71
        assert list(cont) == list(range(off, off + nbytes - 1)), r


@pytest.mark.gpu
def test_canonical_orientation(hip):
    spec, _ = _layers()
    H, L = _pair(hip, spec)
    c, _w = L.decode_scattered()
    assert np.array_equal(c, H.decode_cols())
    n_in, n_out = spec[0], spec[1]
    for B in BATCHES:
        rng = np.random.default_rng(B)
        x = rng.normal(size=(B, n_in)).astype(np.float32)
        g = rng.normal(size=(B, n_out)).astype(np.float32)
        L.forward_dense(x)
        dx = L.backward_dense(g, 0.0)
        assert_close_terms(dx, H.backward_dense(x, g)[0], H.backward_dense(x, g, absmode=True)[0], f"dx B{B}")
        gs, _ = L.sampled_gradw(x, g)
        assert_close_terms(gs, H.sampled_gradw(x, g)[0], H.sampled_gradw(x, g, absmode=True)[0], f"gw B{B}")


@pytest.mark.gpu
def test_shadow_orientation(hip):
    _, spec = _layers()
    H, L = _pair(hip, spec)
    n_in = spec[0]
    for B in BATCHES:
        x = np.random.default_rng(100 + B).normal(size=(B, n_in)).astype(np.float32)
        y = L.forward_dense(x)
        assert_close_terms(y, H.forward_dense(x), H.forward_dense(x, absmode=True), f"fwd B{B}")
