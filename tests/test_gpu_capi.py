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
        L.sili_load_weights.argtypes = [vp, vp, vp, vp, vp, C.c_int64]
        L.sili_backward_dense_train.argtypes = [vp, vp, vp, C.c_int64, vp, C.c_float, C.c_int, C.c_int, C.c_float,
                                                C.c_float, vp]
        L.sili_set_stochastic_rounding.argtypes = [vp, C.c_int]
        L.sili_get_scale_state.argtypes = [vp, vp, vp, vp, vp, vp]
        L.sili_export_scattered.argtypes = [vp, vp, vp, vp, vp]
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
        # learning_rate != 0 runs the optimizer update, which has no sampled grad-W output
        rc = api.L.sili_backward_dense(h, dev["x"], dev["g"], wl.batch, dev["dx"], dev["gw"], None, 0.01, st)
        assert rc == 1 and b"learning_rate == 0" in api.L.sili_last_error()
        for p in dev.values():
            api.ck(api.L.sili_device_free(h, p))
    finally:
        api.L.sili_destroy(h)


def test_capi_backward_dense_train(api):
    """The optimizer update through the C ABI (device buffers, the layer's
    stream, deterministic rounding) against the IEEE restatement: value bytes
    and scale state exact at batch 1, dx within the bar."""
    from train_util import dx_bound, host_layer as train_host, make_train_case
    c = make_train_case(120, 90, 0.1, 77, imp_scales=True)
    H = train_host(c)
    h = C.c_void_p()
    api.ck(api.L.sili_create(c["n_in"], c["n_out"], len(c["cols"]), 0, C.byref(h)))
    dev = {}
    try:
        ptrs, cols, w, imp = (np.ascontiguousarray(c[k]) for k in ("ptrs", "cols", "w", "imp"))
        api.ck(api.L.sili_load_weights(h, _ptr(ptrs), _ptr(cols), _ptr(w), _ptr(imp), len(cols)))
        vs = np.ascontiguousarray(c["vs"])
        api.ck(api.L.sili_set_value_scale(h, _ptr(vs)))
        for name, arr in (("importance", c["is"]), ("output_importance", c["ois"])):
            f = getattr(api.L, f"sili_set_{name}_scale")
            f.argtypes = [C.c_void_p, C.c_void_p]
            api.ck(f(h, _ptr(np.ascontiguousarray(arr))))
        api.ck(api.L.sili_set_stochastic_rounding(h, 0))
        for k, n in (("x", c["n_in"]), ("g", c["n_out"]), ("dx", c["n_in"])):
            dev[k] = C.c_void_p()
            api.ck(api.L.sili_device_alloc(h, n * 4, C.byref(dev[k])))
        st = api.L.sili_stream(h)
        nnz = len(cols)
        for step in range(3):
            x = c["rng"].normal(size=(1, c["n_in"])).astype(np.float32)
            dy = c["rng"].normal(size=(1, c["n_out"])).astype(np.float32)
            api.ck(api.L.sili_memcpy_h2d(h, dev["x"], _ptr(x), x.nbytes))
            api.ck(api.L.sili_memcpy_h2d(h, dev["g"], _ptr(dy), dy.nbytes))
            bound = dx_bound(H, dy, 0.05)
            api.ck(api.L.sili_backward_dense_train(h, dev["x"], dev["g"], 1, dev["dx"], 0.05, 0, 1, 0.999, 1e-8, st))
            api.ck(api.L.sili_synchronize(h))
            dxh, _, _ = H.backward_train(x, dy, 0.05)
            dx = np.zeros_like(x)
            api.ck(api.L.sili_memcpy_d2h(h, _ptr(dx), dev["dx"], dx.nbytes))
            val = np.zeros(nnz, np.uint8)
            api.ck(api.L.sili_export_scattered(h, None, None, None, _ptr(val)))
            assert np.array_equal(val, H.val[:nnz]), f"value bytes, step {step}"
            assert_close_terms(dx, dxh, bound, f"dx, step {step}")
            vsg = np.zeros_like(vs)
            api.ck(api.L.sili_get_value_scale(h, _ptr(vsg)))
            vi, vm = np.zeros_like(vs), np.zeros_like(vs)
            vstep = np.zeros(len(vs), np.uint32)
            api.ck(api.L.sili_get_scale_state(h, _ptr(vi), None, _ptr(vm), _ptr(vstep), None))
            assert np.array_equal(vsg, H.value_scale) and np.array_equal(vi, H.vs_importance)
            assert np.array_equal(vstep, H.vs_step) and np.array_equal(vm, H.vs_momentum)
    finally:
        for p in dev.values():
            api.L.sili_device_free(h, p)
        api.L.sili_destroy(h)


def _capi_layer(api, wl):
    h = C.c_void_p()
    n_b4 = 0 if wl.tile_br is None else 16 * len(wl.tile_br)
    api.ck(api.L.sili_create(wl.n_in, wl.n_out, max(1, wl.nnz + n_b4), 0, C.byref(h)))
    if wl.cols is not None:
        ptrs, cols, q = (np.ascontiguousarray(a) for a in (wl.ptrs, wl.cols, wl.q))
        api.ck(api.L.sili_load_weights(h, _ptr(ptrs), _ptr(cols), _ptr(q), None, wl.nnz))
    if wl.tile_br is not None:
        api.L.sili_load_block4_tiles.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int64]
        br, bc, tb = (np.ascontiguousarray(a) for a in (wl.tile_br, wl.tile_bc, wl.tile_bytes))
        api.ck(api.L.sili_load_block4_tiles(h, _ptr(br), _ptr(bc), _ptr(tb), len(br)))
    vs = np.ascontiguousarray(wl.value_scale, dtype=np.float32)
    api.ck(api.L.sili_set_value_scale(h, _ptr(vs)))
    return h


@pytest.mark.parametrize("cfg,scale,batch", [
    (1, 0.125, 1), (1, 0.125, 4), (1, 0.125, 8), (1, 0.125, 12), (1, 0.125, 64), (1, 0.125, 128),
    (1, 0.125, 256), (1, 0.125, 512), (1, 0.125, 516), (1, 0.125, 6),
    (2, 0.0625, 32), (2, 0.0625, 64), (3, 0.03125, 64)])
def test_capi_backward_with_gradw(api, cfg, scale, batch):
    """backward_dense with grad-W buffers: the fused grad-input + grad-W pass
    (B % 4 == 0, B <= 512) and the separate kernels otherwise."""
    wl = make_config(cfg, scale=scale, batch=batch)
    if wl.g is None:
        wl.g = np.random.default_rng(cfg).normal(size=(batch, wl.n_out)).astype(np.float32)
    H = host_layer(wl)
    h = _capi_layer(api, wl)
    try:
        n_s = max(1, wl.nnz)
        n_b = 0 if wl.tile_br is None else 16 * len(wl.tile_br)
        dev = {}
        for name, n in (("x", wl.x.size), ("g", wl.g.size), ("y", batch * wl.n_out),
                        ("dx", batch * wl.n_in), ("gws", n_s), ("gwb", max(1, n_b))):
            p = C.c_void_p()
            api.ck(api.L.sili_device_alloc(h, 4 * n, C.byref(p)))
            dev[name] = p
        x = np.ascontiguousarray(wl.x, dtype=np.float32)
        g = np.ascontiguousarray(wl.g, dtype=np.float32)
        api.ck(api.L.sili_memcpy_h2d(h, dev["x"], _ptr(x), x.nbytes))
        api.ck(api.L.sili_memcpy_h2d(h, dev["g"], _ptr(g), g.nbytes))
        st = api.L.sili_stream(h)
        api.ck(api.L.sili_forward_dense(h, dev["x"], batch, dev["y"], st))
        api.ck(api.L.sili_backward_dense(h, dev["x"], dev["g"], batch, dev["dx"], dev["gws"],
                                         dev["gwb"] if n_b else None, 0.0, st))
        api.ck(api.L.sili_synchronize(h))
        dx = np.zeros((batch, wl.n_in), np.float32)
        api.ck(api.L.sili_memcpy_d2h(h, _ptr(dx), dev["dx"], dx.nbytes))
        dx_o, ai_o, ag_o = H.backward_dense(x, g)
        assert_close_terms(dx, dx_o, H.backward_dense(x, g, absmode=True)[0], "dx")
        gs_o, gb_o = H.sampled_gradw(x, g)
        gs_a, gb_a = H.sampled_gradw(x, g, absmode=True)
        if wl.nnz:
            gs = np.zeros(wl.nnz, np.float32)
            api.ck(api.L.sili_memcpy_d2h(h, _ptr(gs), dev["gws"], gs.nbytes))
            assert_close_terms(gs, gs_o, gs_a, "gw scattered")
        if n_b:
            gb = np.zeros(n_b, np.float32)
            api.ck(api.L.sili_memcpy_d2h(h, _ptr(gb), dev["gwb"], gb.nbytes))
            assert_close_terms(gb, gb_o, gb_a, "gw block4")
        ai = np.zeros(wl.n_in, np.float32)
        ag = np.zeros(wl.n_out, np.float32)
        api.ck(api.L.sili_get_accumulators(h, _ptr(ai), _ptr(ag)))
        assert_close_terms(ai, ai_o, ai_o, "acc_in")
        assert_close_terms(ag, ag_o, ag_o, "acc_grad")
        for p in dev.values():
            api.ck(api.L.sili_device_free(h, p))
    finally:
        api.L.sili_destroy(h)


def test_capi_profiler_names_and_counts(api):
    """Per-kernel times come from the dispatches' own begin/end stamps."""
    wl = make_config(1, scale=0.125, batch=64)
    h = _capi_layer(api, wl)

    class Entry(C.Structure):
        _fields_ = [("name", C.c_char * 56), ("count", C.c_int64), ("total_ms", C.c_double),
                    ("min_ms", C.c_double), ("max_ms", C.c_double)]
    api.L.sili_profile_read.argtypes = [C.c_void_p, C.POINTER(Entry), C.c_int, C.POINTER(C.c_int)]
    try:
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
        for _ in range(3):
            api.ck(api.L.sili_forward_dense(h, dev["x"], wl.batch, dev["y"], st))
            api.ck(api.L.sili_backward_dense(h, None, dev["g"], wl.batch, dev["dx"], dev["gw"], None, 0.0, st))
        api.ck(api.L.sili_synchronize(h))
        buf = (Entry * 64)()
        n = C.c_int()
        api.ck(api.L.sili_profile_read(h, buf, 64, C.byref(n)))
        got = {buf[i].name.decode(): (buf[i].count, buf[i].total_ms, buf[i].min_ms) for i in range(n.value)}
        for name in ("fwd:transpose", "fwd:gather", "bwd:transpose", "bwd:gather_gradw"):
            assert name in got, got
            cnt, tot, mn = got[name]
            assert cnt == 3 and tot > 0 and mn > 0, (name, got[name])
        assert "bwd:gather" not in got and "bwd:sddmm" not in got
        for p in dev.values():
            api.ck(api.L.sili_device_free(h, p))
    finally:
        api.L.sili_destroy(h)


@pytest.mark.parametrize("offset", [0, 1, 4, 12])
def test_capi_ordered_copies_page_locked(api, offset):
    """sili_memcpy_h2d_ordered / _d2h_ordered between device memory and
    page-locked host memory (sili_host_alloc) run as a copy kernel on the
    layer's stream: every byte arrives for sizes with 16-, 4- and 1-byte
    tails at 16-, 4- and 1-byte host offsets; pageable memory takes the
    runtime's copy and gives the same bytes."""
    vp = C.c_void_p
    L = api.L
    L.sili_host_alloc.argtypes = [C.c_size_t, C.POINTER(vp)]
    L.sili_host_free.argtypes = [vp]
    L.sili_memcpy_h2d_ordered.argtypes = [vp, vp, vp, C.c_size_t]
    L.sili_memcpy_d2h_ordered.argtypes = [vp, vp, vp, C.c_size_t]
    h = vp()
    api.ck(L.sili_create(64, 64, 16, 0, C.byref(h)))
    cap = (3 << 20) + 64
    hp, dv = vp(), vp()
    try:
        api.ck(L.sili_host_alloc(cap, C.byref(hp)))
        api.ck(L.sili_device_alloc(h, cap, C.byref(dv)))
        host = np.ctypeslib.as_array(C.cast(hp, C.POINTER(C.c_uint8)), shape=(cap,))
        rng = np.random.default_rng(7 + offset)
        for nbytes in (1, 3, 17, 64, 1000, 65536 + 5, (2 << 20) + 13, 3 << 20):
            src = rng.integers(0, 256, nbytes, dtype=np.uint8)
            host[:] = 0
            host[offset:offset + nbytes] = src
            api.ck(L.sili_memcpy_h2d_ordered(h, dv, hp.value + offset, nbytes))
            # back through pageable memory (the runtime's copy) ...
            back = np.zeros(nbytes, np.uint8)
            api.ck(L.sili_memcpy_d2h_ordered(h, _ptr(back), dv, nbytes))
            assert np.array_equal(back, src), nbytes
            # ... and through the page-locked block at another offset
            host[:] = 0
            o2 = (offset + 3) % 16
            api.ck(L.sili_memcpy_d2h_ordered(h, hp.value + o2, dv, nbytes))
            assert np.array_equal(host[o2:o2 + nbytes], src), nbytes
            assert not host[:o2].any() and not host[o2 + nbytes:].any(), nbytes
            # pageable source, page-locked destination
            src2 = src[::-1].copy()
            api.ck(L.sili_memcpy_h2d_ordered(h, dv, _ptr(src2), nbytes))
            api.ck(L.sili_memcpy_d2h_ordered(h, hp.value, dv, nbytes))
            assert np.array_equal(host[:nbytes], src2), nbytes
        del host
    finally:
        if dv.value:
            L.sili_device_free(h, dv)
        if hp.value:
            L.sili_host_free(hp)
        L.sili_destroy(h)
