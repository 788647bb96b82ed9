"""GPU tests that drive the C ABI directly through ctypes (no pybind layer):
device buffers, explicit streams, the NULL-x backward (stored forward input)
and the profiler entry points."""
import ctypes as C

import numpy as np
import pytest

from sili__new_amd.synth import make_config
from tests.util import assert_close_terms, host_layer

pytestmark = pytest.mark.gpu


class Api:
    def __init__(self, path):
        L = C.CDLL(path)
        vp = C.c_void_p
        L.sili_last_error.restype = C.c_char_p
        L.sili_create.argtypes = [C.c_int64, C.c_int64, C.c_int64, C.c_int, C.POINTER(vp)]
        L.sili_destroy.argtypes = [vp]
        L.sili_load_weights.argtypes = [vp, vp, vp, vp, vp, C.c_int64]
        L.sili_set_value_scale.argtypes = [vp, vp]
        L.sili_forward_dense.argtypes = [vp, vp, C.c_int64, vp, vp]
        L.sili_backward_dense.argtypes = [vp, vp, vp, C.c_int64, vp, vp, vp, C.c_float, vp]
        L.sili_device_alloc.argtypes = [vp, C.c_size_t, C.POINTER(vp)]
        L.sili_device_free.argtypes = [vp, vp]
        L.sili_memcpy_h2d.argtypes = [vp, vp, vp, C.c_size_t]
        L.sili_memcpy_d2h.argtypes = [vp, vp, vp, C.c_size_t]
        L.sili_synchronize.argtypes = [vp]
        L.sili_stream.restype = vp
        L.sili_stream.argtypes = [vp]
        L.sili_get_accumulators.argtypes = [vp, vp, vp]
        L.sili_zero_accum.argtypes = [vp]
        L.sili_profile_enable.argtypes = [vp, C.c_int]
        self.L = L

    def ck(self, rc):
        assert rc == 0, self.L.sili_last_error().decode()


def _ptr(a):
    return a.ctypes.data_as(C.c_void_p)


@pytest.fixture()
def api(hip):
    return Api(hip.LIB_PATH)


def test_capi_forward_backward_null_x(api):
    wl = make_config(1, scale=0.125, batch=64)
    H = host_layer(wl)
    h = C.c_void_p()
    api.ck(api.L.sili_create(wl.n_in, wl.n_out, wl.nnz, 0, C.byref(h)))
    try:
        ptrs, cols, q = (np.ascontiguousarray(a) for a in (wl.ptrs, wl.cols, wl.q))
        api.ck(api.L.sili_load_weights(h, _ptr(ptrs), _ptr(cols), _ptr(q), None, wl.nnz))
        vs = np.ascontiguousarray(wl.value_scale)
        api.ck(api.L.sili_set_value_scale(h, _ptr(vs)))
        dev = {}
        for name, n in (("x", wl.x.size), ("g", wl.g.size), ("y", wl.batch * wl.n_out),
                        ("dx", wl.batch * wl.n_in), ("gw", wl.nnz)):
            p = C.c_void_p()
            api.ck(api.L.sili_device_alloc(h, 4 * n, C.byref(p)))
            dev[name] = p
        api.ck(api.L.sili_memcpy_h2d(h, dev["x"], _ptr(wl.x), wl.x.nbytes))
        api.ck(api.L.sili_memcpy_h2d(h, dev["g"], _ptr(wl.g), wl.g.nbytes))
        st = api.L.sili_stream(h)
        api.ck(api.L.sili_profile_enable(h, 1))
        api.ck(api.L.sili_forward_dense(h, dev["x"], wl.batch, dev["y"], st))
        # NULL x: the stored forward input is used (batch > 1)
        api.ck(api.L.sili_backward_dense(h, None, dev["g"], wl.batch, dev["dx"], dev["gw"], None, 0.0, st))
        api.ck(api.L.sili_synchronize(h))
        y = np.zeros((wl.batch, wl.n_out), np.float32)
        dx = np.zeros((wl.batch, wl.n_in), np.float32)
        gw = np.zeros(wl.nnz, np.float32)
        api.ck(api.L.sili_memcpy_d2h(h, _ptr(y), dev["y"], y.nbytes))
        api.ck(api.L.sili_memcpy_d2h(h, _ptr(dx), dev["dx"], dx.nbytes))
        api.ck(api.L.sili_memcpy_d2h(h, _ptr(gw), dev["gw"], gw.nbytes))
        assert_close_terms(y, H.forward_dense(wl.x), H.forward_dense(wl.x, absmode=True), "y")
        dx_o, ai_o, ag_o = H.backward_dense(wl.x, wl.g)
        assert_close_terms(dx, dx_o, H.backward_dense(wl.x, wl.g, absmode=True)[0], "dx")
        assert_close_terms(gw, H.sampled_gradw(wl.x, wl.g)[0], H.sampled_gradw(wl.x, wl.g, absmode=True)[0], "gw")
        ai = np.zeros(wl.n_in, np.float32)
        ag = np.zeros(wl.n_out, np.float32)
        api.ck(api.L.sili_get_accumulators(h, _ptr(ai), _ptr(ag)))
        assert_close_terms(ai, ai_o, ai_o, "acc_in (fused in grad-W)")
        assert_close_terms(ag, ag_o, ag_o, "acc_grad")
        # batch mismatch with a NULL x is an error, not a silent reuse
        rc = api.L.sili_backward_dense(h, None, dev["g"], 32, dev["dx"], None, None, 0.0, st)
        assert rc == 1 and b"stored" in api.L.sili_last_error()
        # learning_rate != 0 is rejected (optimizer update not on the GPU path)
        rc = api.L.sili_backward_dense(h, dev["x"], dev["g"], wl.batch, dev["dx"], None, None, 0.01, st)
        assert rc == 1
        for p in dev.values():
            api.ck(api.L.sili_device_free(h, p))
    finally:
        api.L.sili_destroy(h)
