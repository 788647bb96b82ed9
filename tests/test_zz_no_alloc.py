"""GPU: sili_forward_dense_noalloc through the C ABI (ctypes) against
sili_forward_dense on the same layer and input: two calls in a row, the
second with a smaller input, within the fp32 bar of the oracle's term sums;
the scratch limit turned into an error before any device work; pending
synaptogenesis policy edits refused (writing them allocates) until
sili_synchronize writes them; and the device's free memory unchanged across
repeated calls."""
import ctypes as C

import numpy as np
import pytest

from sili__new_amd.synth import make_config
from tests.util import assert_close_terms, host_layer

pytestmark = pytest.mark.gpu

SILI_ERR_INVALID = 1
SCRATCH_FLOATS = (32 << 20) // 4


class Api:
    def __init__(self, path):
        L = C.CDLL(path)
        vp = C.c_void_p
        L.sili_last_error.restype = C.c_char_p
        L.sili_create.argtypes = [C.c_int64, C.c_int64, C.c_int64, C.c_int, C.POINTER(vp)]
        L.sili_destroy.argtypes = [vp]
        L.sili_load_weights.argtypes = [vp, vp, vp, vp, vp, C.c_int64]
        L.sili_load_block4_tiles.argtypes = [vp, vp, vp, vp, C.c_int64]
        L.sili_set_value_scale.argtypes = [vp, vp]
        L.sili_forward_dense.argtypes = [vp, vp, C.c_int64, vp, vp]
        L.sili_forward_dense_noalloc.argtypes = [vp, vp, C.c_int64, vp, vp]
        L.sili_device_alloc.argtypes = [vp, C.c_size_t, C.POINTER(vp)]
        L.sili_device_free.argtypes = [vp, vp]
        L.sili_memcpy_h2d.argtypes = [vp, vp, vp, C.c_size_t]
        L.sili_memcpy_d2h.argtypes = [vp, vp, vp, C.c_size_t]
        L.sili_memset_device.argtypes = [vp, vp, C.c_int, C.c_size_t]
        L.sili_synchronize.argtypes = [vp]
        L.sili_backward_dense.argtypes = [vp, vp, vp, C.c_int64, vp, vp, vp, C.c_float, vp]
        L.sili_build_probes.argtypes = [vp, C.c_int64, C.c_int]
        L.sili_synap_step.argtypes = [vp, C.c_float, C.c_int64, C.c_int64, C.c_float, C.POINTER(C.c_int)]
        L.sili_get_info.argtypes = [vp, vp]
        L.sili_stream.restype = vp
        L.sili_stream.argtypes = [vp]
        self.L = L

    def ck(self, rc):
        assert rc == 0, self.L.sili_last_error().decode()


def _ptr(a):
    return a.ctypes.data_as(C.c_void_p)


@pytest.fixture()
def api(hip):
    return Api(hip.LIB_PATH)


def _layer(api, wl):
    h = C.c_void_p()
    n_tiles = 0 if wl.tile_br is None else len(wl.tile_br)
    api.ck(api.L.sili_create(wl.n_in, wl.n_out, max(1, wl.nnz + 16 * n_tiles), 0, C.byref(h)))
    if wl.cols is not None:
        ptrs, cols, q = (np.ascontiguousarray(a) for a in (wl.ptrs, wl.cols, wl.q))
        api.ck(api.L.sili_load_weights(h, _ptr(ptrs), _ptr(cols), _ptr(q), None, wl.nnz))
    if wl.tile_br is not None:
        br = np.ascontiguousarray(wl.tile_br, np.int32)
        bc = np.ascontiguousarray(wl.tile_bc, np.int32)
        tb = np.ascontiguousarray(wl.tile_bytes, np.uint8)
        api.ck(api.L.sili_load_block4_tiles(h, _ptr(br), _ptr(bc), _ptr(tb), len(br)))
    vs = np.ascontiguousarray(wl.value_scale, np.float32)
    api.ck(api.L.sili_set_value_scale(h, _ptr(vs)))
    return h


def _alloc(api, h, nbytes):
    p = C.c_void_p()
    api.ck(api.L.sili_device_alloc(h, nbytes, C.byref(p)))
    return p


@pytest.mark.parametrize("cfg,scale,batches", [(1, 0.25, (64, 16)), (1, 0.25, (8, 1)), (3, 0.0625, (32, 5)),
                                               (2, 0.0625, (100, 64))])
def test_noalloc_forward_matches_forward_dense(api, cfg, scale, batches):
    wl = make_config(cfg, scale=scale, batch=max(batches))
    H = host_layer(wl)
    h = _layer(api, wl)
    bufs = []
    try:
        st = api.L.sili_stream(h)
        for B in batches:
            x = np.ascontiguousarray(wl.x[:B], np.float32)
            dx_, dy1, dy2 = (_alloc(api, h, n) for n in (x.nbytes, 4 * B * wl.n_out, 4 * B * wl.n_out))
            bufs += [dx_, dy1, dy2]
            api.ck(api.L.sili_memcpy_h2d(h, dx_, _ptr(x), x.nbytes))
            # outputs start as garbage: the entry point overwrites every element
            api.ck(api.L.sili_memset_device(h, dy2, 0x7F, 4 * B * wl.n_out))
            api.ck(api.L.sili_forward_dense(h, dx_, B, dy1, st))
            api.ck(api.L.sili_forward_dense_noalloc(h, dx_, B, dy2, st))
            api.ck(api.L.sili_synchronize(h))
            y1 = np.zeros((B, wl.n_out), np.float32)
            y2 = np.zeros((B, wl.n_out), np.float32)
            api.ck(api.L.sili_memcpy_d2h(h, _ptr(y1), dy1, y1.nbytes))
            api.ck(api.L.sili_memcpy_d2h(h, _ptr(y2), dy2, y2.nbytes))
            bound = H.forward_dense(x, absmode=True)
            assert_close_terms(y2, y1, 2 * bound, f"noalloc vs forward_dense c{cfg} B{B}")
            assert_close_terms(y2, H.forward_dense(x), bound, f"noalloc vs oracle c{cfg} B{B}")
    finally:
        for p in bufs:
            api.L.sili_device_free(h, p)
        api.L.sili_destroy(h)


def test_noalloc_rejects_inputs_beyond_the_scratch(api):
    n_in, n_out = 8192, 16
    B = SCRATCH_FLOATS // n_in + 1
    h = C.c_void_p()
    api.ck(api.L.sili_create(n_in, n_out, 1, 0, C.byref(h)))
    try:
        x = _alloc(api, h, 4 * B * n_in)
        y = _alloc(api, h, 4 * B * n_out)
        rc = api.L.sili_forward_dense_noalloc(h, x, B, y, None)
        assert rc == SILI_ERR_INVALID
        assert b"scratch" in api.L.sili_last_error()
        # the largest batch that fits is accepted
        api.ck(api.L.sili_forward_dense_noalloc(h, x, B - 1, y, None))
        api.ck(api.L.sili_synchronize(h))
        api.L.sili_device_free(h, x)
        api.L.sili_device_free(h, y)
    finally:
        api.L.sili_destroy(h)


def _mem_free():
    hip_rt = C.CDLL("libamdhip64.so")
    free, total = C.c_size_t(), C.c_size_t()
    assert hip_rt.hipMemGetInfo(C.byref(free), C.byref(total)) == 0
    return free.value


def test_noalloc_refuses_pending_policy_edits(api):
    """A synap_step leaves its edits pending on the host; noalloc refuses to
    write them (that allocates), sili_synchronize writes them, and noalloc
    then equals forward_dense on the edited layer.  Every buffer is
    allocated and filled before the policy calls: those entry points write
    pending edits too."""
    wl = make_config(1, scale=0.125, batch=16)
    h = _layer(api, wl)
    bufs = []
    try:
        B = wl.batch
        x = np.ascontiguousarray(wl.x, np.float32)
        g = np.ascontiguousarray(wl.g, np.float32)
        dxx, dgg, ddx, dy1, dy2 = (_alloc(api, h, n) for n in (x.nbytes, g.nbytes, 4 * B * wl.n_in,
                                                             4 * B * wl.n_out, 4 * B * wl.n_out))
        bufs += [dxx, dgg, ddx, dy1, dy2]
        api.ck(api.L.sili_memcpy_h2d(h, dxx, _ptr(x), x.nbytes))
        api.ck(api.L.sili_memcpy_h2d(h, dgg, _ptr(g), g.nbytes))
        # the accumulators the probes rank by
        api.ck(api.L.sili_backward_dense(h, dxx, dgg, B, ddx, None, None, 0.0, None))

        def outputs():
            y1 = np.zeros((B, wl.n_out), np.float32)
            y2 = np.zeros((B, wl.n_out), np.float32)
            api.ck(api.L.sili_memcpy_d2h(h, _ptr(y1), dy1, y1.nbytes))
            api.ck(api.L.sili_memcpy_d2h(h, _ptr(y2), dy2, y2.nbytes))
            return y1, y2

        did = C.c_int()
        for sync in (False, True):
            api.ck(api.L.sili_build_probes(h, 4, 0))
            # importance nibbles are 0 after load_weights: every row prunes
            api.ck(api.L.sili_synap_step(h, 0.5, 1 << 20, 8, 1e-3, C.byref(did)))
            assert did.value == 1
            if not sync:
                rc = api.L.sili_forward_dense_noalloc(h, dxx, B, dy2, None)
                assert rc == SILI_ERR_INVALID
                assert b"pending" in api.L.sili_last_error()
            api.ck(api.L.sili_synchronize(h))  # writes the edits
            api.ck(api.L.sili_memset_device(h, dy2, 0x7F, 4 * B * wl.n_out))
            api.ck(api.L.sili_forward_dense_noalloc(h, dxx, B, dy2, None))
            api.ck(api.L.sili_forward_dense(h, dxx, B, dy1, None))
            api.ck(api.L.sili_synchronize(h))
            y1, y2 = outputs()
            # the two paths may sum in different orders; a stale or
            # unwritten output would be far outside this
            assert np.allclose(y2, y1, rtol=1e-5, atol=1e-6 * np.abs(y1).max()), sync
    finally:
        for p in bufs:
            api.L.sili_device_free(h, p)
        api.L.sili_destroy(h)


def test_noalloc_leaves_free_device_memory_unchanged(api):
    wl = make_config(3, scale=0.0625, batch=32)
    h = _layer(api, wl)
    bufs = []
    try:
        st = api.L.sili_stream(h)
        x = np.ascontiguousarray(wl.x, np.float32)
        dx_, dy = _alloc(api, h, x.nbytes), _alloc(api, h, 4 * wl.batch * wl.n_out)
        bufs += [dx_, dy]
        api.ck(api.L.sili_memcpy_h2d(h, dx_, _ptr(x), x.nbytes))
        api.ck(api.L.sili_forward_dense_noalloc(h, dx_, wl.batch, dy, st))
        api.ck(api.L.sili_synchronize(h))
        before = _mem_free()
        for B in (32, 7, 32, 1, 16):
            api.ck(api.L.sili_forward_dense_noalloc(h, dx_, B, dy, st))
        api.ck(api.L.sili_synchronize(h))
        assert _mem_free() == before
    finally:
        for p in bufs:
            api.L.sili_device_free(h, p)
        api.L.sili_destroy(h)
