"""Arrays the pybind module returns live in page-locked host blocks.

The module hands its outputs back in blocks from a process-wide pool (each
array holds its block until it dies) and uploads its inputs on the layer's
stream.  Checked here: an output stays valid and writable after its layer is
gone, an output passed back as an input (the page-locked, DMA path) gives
the same result as a plain numpy copy of it (the staged path), blocks are
reused after their arrays die, and the results match the oracle.
"""
from __future__ import annotations

import gc

import numpy as np
import pytest

from sili__new_amd.synth import make_config
from tests.util import assert_close_terms, host_layer, gpu_layer

pytestmark = pytest.mark.gpu


def test_outputs_outlive_layer_and_chain(hip):
    wl = make_config(1, scale=0.125, batch=16)
    H = host_layer(wl)
    L = gpu_layer(hip, wl)
    y = L.forward_dense(wl.x)
    assert y.flags.c_contiguous and y.flags.writeable and y.dtype == np.float32
    assert_close_terms(y, H.forward_dense(wl.x), H.forward_dense(wl.x, absmode=True), "forward")
    # an output as the next call's input (page-locked source) and a plain copy
    # of it (pageable source) give the same bytes
    y2_pinned = L.forward_dense(y)
    y2_plain = L.forward_dense(np.array(y, copy=True))
    assert np.array_equal(y2_pinned, y2_plain)
    dx_pinned = L.backward_dense(y, 0.0)
    dx_plain = L.backward_dense(np.array(y, copy=True), 0.0)
    np.testing.assert_allclose(dx_pinned, dx_plain, rtol=1e-6, atol=0)
    gs, gb = L.sampled_gradw(y, y)
    gs2, _ = L.sampled_gradw(np.array(y), np.array(y))
    np.testing.assert_allclose(gs, gs2, rtol=1e-6, atol=0)
    keep = y.copy()
    del L
    gc.collect()
    # the array still owns its block
    assert np.array_equal(y, keep)
    y[0, 0] = 123.0
    assert y[0, 0] == 123.0


def test_blocks_reused_after_arrays_die(hip):
    wl = make_config(1, scale=0.125, batch=16)
    L = gpu_layer(hip, wl)
    want = L.forward_dense(wl.x).copy()
    addrs = set()
    for _ in range(50):
        y = L.forward_dense(wl.x)
        addrs.add(y.ctypes.data)
        assert np.array_equal(y, want)
        del y
        gc.collect()
    # a block freed by a dead array is taken by the next output
    assert len(addrs) <= 2
    # many live outputs at once each get their own block
    live = [L.forward_dense(wl.x) for _ in range(8)]
    assert len({a.ctypes.data for a in live}) == 8
    for a in live:
        assert np.array_equal(a, want)


def test_interior_and_staged_inputs(hip):
    """Inputs that start inside a returned (page-locked) array, at 4- and
    16-byte offsets, and ordinary numpy inputs above the 64 KiB staging size
    give the bytes a plain copy of them gives, on every path that uploads."""
    wl = make_config(1, scale=0.125, batch=16)
    assert wl.n_in == wl.n_out
    L = gpu_layer(hip, wl)
    big = L.forward_dense(np.concatenate([wl.x, wl.x]))  # 32 rows, page-locked
    flat = big.reshape(-1)
    n = wl.n_in
    for off in (1, 4, n):
        xin = flat[off:off + 16 * n].reshape(16, n)
        assert not xin.flags.owndata
        y_a = L.forward_dense(xin)
        y_b = L.forward_dense(np.array(xin, copy=True))
        assert np.array_equal(y_a, y_b), off
        # (split rows add their partial sums atomically: same values to 1e-6)
        dx_a = L.backward_dense(xin, 0.0)
        dx_b = L.backward_dense(np.array(xin, copy=True), 0.0)
        np.testing.assert_allclose(dx_a, dx_b, rtol=1e-6, atol=0, err_msg=str(off))
        gs_a, gb_a = L.sampled_gradw(xin, xin)
        gs_b, gb_b = L.sampled_gradw(np.array(xin), np.array(xin))
        np.testing.assert_allclose(gs_a, gs_b, rtol=1e-6, atol=0, err_msg=str(off))
        np.testing.assert_allclose(gb_a, gb_b, rtol=1e-6, atol=0, err_msg=str(off))
    H = host_layer(wl)
    y = L.forward_dense(wl.x)
    assert_close_terms(y, H.forward_dense(wl.x), H.forward_dense(wl.x, absmode=True), "forward")
