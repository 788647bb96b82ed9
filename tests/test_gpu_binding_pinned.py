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
