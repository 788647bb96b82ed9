"""Split rows summed in item order (SILI_SPLIT_COMBINE=1 when the store is
built): rows longer than one work item are combined by the last of their
items to finish, from per-item partial sums, instead of with float atomics.

A layer with split rows in both orientations (one input row of 2000
synapses: the canonical store; one output column fed by every input: the
shadow store) -- the forward gather, the grad-input gather and the fused
grad-input + sampled grad-W kernel against the oracle, and each output
bitwise equal over repeated calls.  The same layer built with atomics must
agree with it within the fp32 bar.
"""
import ctypes as C

import numpy as np
import pytest

from oracle import HostLayer
from tests.test_gpu_capi import Api, _ptr
from tests.util import assert_close_terms

pytestmark = pytest.mark.gpu


def _skewed(seed, n_in=4096, n_out=2048):
    rng = np.random.default_rng(seed)
    rows = []
    for r in range(n_in):
        k = 2000 if r == 3 else int(rng.integers(1, 60))
        c = set(rng.choice(n_out, k, replace=False).tolist())
        c.add(7)  # output 7 is fed by every input: its shadow row is split too
        rows.append(sorted(c))
    ptrs = np.zeros(n_in + 1, np.int32)
    ptrs[1:] = np.cumsum([len(r) for r in rows])
    cols = np.concatenate(rows).astype(np.int32)
    w = rng.normal(0.0, 2.0, len(cols)).astype(np.float32)
    return n_in, n_out, ptrs, cols, w


def _layers(hip, monkeypatch, combine):
    n_in, n_out, ptrs, cols, w = _skewed(11)
    monkeypatch.setenv("SILI_SPLIT_COMBINE", "1" if combine else "0")
    L = hip.SparseLinearLayer(n_in, n_out, len(cols))
    L.load_weights(ptrs, cols, w)
    H = HostLayer(n_in, n_out).load_csr(ptrs, cols, w=w)
    return L, H, n_in, n_out, len(cols)


@pytest.mark.parametrize("B", [12, 32, 64])
def test_forward_and_grad_input_combined_in_order(hip, monkeypatch, B):
    L, H, n_in, n_out, _ = _layers(hip, monkeypatch, True)
    info = L.info()
    assert info["split_combined"] == 3, info
    assert info["n_segments"] > n_in
    rng = np.random.default_rng(B)
    x = rng.normal(size=(B, n_in)).astype(np.float32)
    g = rng.normal(size=(B, n_out)).astype(np.float32)
    y = L.forward_dense(x)
    assert_close_terms(y, H.forward_dense(x), H.forward_dense(x, absmode=True), "y")
    dx = L.backward_dense(g, 0.0)
    assert_close_terms(dx, H.backward_dense(x, g)[0], H.backward_dense(x, g, absmode=True)[0], "dx")
    for _ in range(3):
        assert np.array_equal(L.forward_dense(x).view(np.uint32), y.view(np.uint32))
        assert np.array_equal(L.backward_dense(g, 0.0).view(np.uint32), dx.view(np.uint32))
    # the same layer with atomics agrees within the bar
    La, _, _, _, _ = _layers(hip, monkeypatch, False)
    assert La.info()["split_combined"] == 0
    assert_close_terms(La.forward_dense(x), y, H.forward_dense(x, absmode=True), "y atomics")
    assert_close_terms(La.backward_dense(g, 0.0), dx, H.backward_dense(x, g, absmode=True)[0], "dx atomics")


def test_fused_backward_combined_in_order(hip, monkeypatch):
    """k_bwd_v4 (grad-input with the sampled grad-W) through the C ABI."""
    n_in, n_out, ptrs, cols, w = _skewed(12)
    monkeypatch.setenv("SILI_SPLIT_COMBINE", "1")
    api = Api(hip.LIB_PATH)
    H = HostLayer(n_in, n_out).load_csr(ptrs, cols, w=w)
    nnz = len(cols)
    B = 64
    rng = np.random.default_rng(3)
    x = rng.normal(size=(B, n_in)).astype(np.float32)
    g = rng.normal(size=(B, n_out)).astype(np.float32)
    h = C.c_void_p()
    api.ck(api.L.sili_create(n_in, n_out, nnz, 0, C.byref(h)))
    try:
        api.ck(api.L.sili_load_weights(h, _ptr(ptrs), _ptr(cols), _ptr(w), None, nnz))
        dev = {}
        for name, n in (("x", x.size), ("g", g.size), ("dx", B * n_in), ("gw", nnz)):
            p = C.c_void_p()
            api.ck(api.L.sili_device_alloc(h, 4 * n, C.byref(p)))
            dev[name] = p
        api.ck(api.L.sili_memcpy_h2d(h, dev["x"], _ptr(x), x.nbytes))
        api.ck(api.L.sili_memcpy_h2d(h, dev["g"], _ptr(g), g.nbytes))
        st = api.L.sili_stream(h)
        outs = []
        for _ in range(3):
            api.ck(api.L.sili_backward_dense(h, dev["x"], dev["g"], B, dev["dx"], dev["gw"], None, 0.0, st))
            api.ck(api.L.sili_synchronize(h))
            dx = np.zeros((B, n_in), np.float32)
            gw = np.zeros(nnz, np.float32)
            api.ck(api.L.sili_memcpy_d2h(h, _ptr(dx), dev["dx"], dx.nbytes))
            api.ck(api.L.sili_memcpy_d2h(h, _ptr(gw), dev["gw"], gw.nbytes))
            outs.append((dx, gw))
        dx, gw = outs[0]
        assert_close_terms(dx, H.backward_dense(x, g)[0], H.backward_dense(x, g, absmode=True)[0], "fused dx")
        assert_close_terms(gw, H.sampled_gradw(x, g)[0], H.sampled_gradw(x, g, absmode=True)[0], "fused grad-W")
        for dxi, gwi in outs[1:]:
            assert np.array_equal(dxi.view(np.uint32), dx.view(np.uint32))
            assert np.array_equal(gwi.view(np.uint32), gw.view(np.uint32))
        for p in dev.values():
            api.ck(api.L.sili_device_free(h, p))
    finally:
        api.L.sili_destroy(h)
