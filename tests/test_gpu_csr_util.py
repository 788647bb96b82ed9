"""GPU: the module utilities fp4_quantize_array, dense_to_csr and
dense_to_top_k_csr (sili/cpu_backend.cpp:3075-3172) against their oracle
restatements (pinned to the reference's tests and compiled top_k_csr in
tests/test_csr_util_oracle.py), through the pybind module and the raw C ABI."""
import ctypes as C

import numpy as np
import pytest

import oracle
from oracle import lib as olib

pytestmark = pytest.mark.gpu


def test_fp4_quantize_array_on_device(hip):
    v = np.linspace(-8, 8, 4097, dtype=np.float32)
    v = np.concatenate([v, np.float32([np.nan, np.inf, -np.inf, 0.25, -0.25, 0.2499999, 5.0, 1.75])])
    got = np.asarray(hip.fp4_quantize_array(v))
    want = np.array([olib().oracle_fp4_encode(float(x)) for x in v], np.uint8)
    assert np.array_equal(got, want)
    assert hip.fp4_quantize_array(np.zeros(0, np.float32)).size == 0


def _same_csr(a, b, what):
    for u, w, name in zip(a, b, ("ptrs", "indices", "values")):
        u, w = np.asarray(u), np.asarray(w)
        assert u.dtype == w.dtype and np.array_equal(u.view(np.uint8), w.view(np.uint8)), f"{what}: {name}"


@pytest.mark.parametrize("rows,cols,thr", [(2, 3, 0.0), (1, 2, 0.01), (32, 16384, 1.6), (5, 1000, 0.0),
                                           (7, 257, 1e-4), (3, 0, 0.5)])
def test_dense_to_csr_matches_oracle(hip, rows, cols, thr):
    rng = np.random.default_rng(rows * 31 + cols)
    x = rng.normal(size=(rows, cols)).astype(np.float32)
    if cols:
        x[rng.random(x.shape) < 0.3] = 0.0
        x.flat[::97] = -0.0
        x.flat[5::211] = np.nan
        x.flat[7::301] = np.float32(thr)  # at the threshold: not kept
    _same_csr(hip.dense_to_csr(x, thr), oracle.dense_to_csr(x, thr), f"dense_to_csr {rows}x{cols}")
    if rows == 1:
        _same_csr(hip.dense_to_csr(x[0], thr), oracle.dense_to_csr(x[0], thr), "1-D input")


@pytest.mark.parametrize("rows,cols,k", [(1, 100, 7), (4, 33, 20), (32, 16384, 491), (8, 64, 10_000),
                                         (3, 7, 0), (16, 300, 1), (2, 5, 4)])
def test_dense_to_top_k_csr_matches_oracle(hip, rows, cols, k):
    rng = np.random.default_rng(rows * 7 + k)
    x = rng.normal(size=(rows, cols)).astype(np.float32)
    x[rng.random(x.shape) < 0.2] = 0.0
    # ties across the cut: the lowest flat index is kept on both sides
    x.flat[3::50] = np.float32(1.25)
    x.flat[4::50] = np.float32(-1.25)
    _same_csr(hip.dense_to_top_k_csr(x, k, 4), oracle.dense_to_top_k_csr(x, k), f"top-k {rows}x{cols} k={k}")


def test_capi_dense_to_csr_capacity(hip):
    """The raw C ABI reports the count and refuses a too-small capacity
    with SILI_ERR_RANGE (ptrs still written)."""
    L = C.CDLL(hip.LIB_PATH)
    vp = C.c_void_p
    L.sili_buffer_alloc.argtypes = [C.c_int, C.c_size_t, C.POINTER(vp)]
    L.sili_buffer_free.argtypes = [C.c_int, vp]
    L.sili_buffer_copy.argtypes = [C.c_int, vp, vp, C.c_size_t]
    L.sili_dense_to_csr.argtypes = [vp, C.c_int64, C.c_int64, C.c_float, vp, vp, vp, C.c_int64,
                                    C.POINTER(C.c_int64), vp]
    x = np.array([[1.0, 0.0, 2.0], [0.0, 3.0, 0.0]], np.float32)
    bufs = []

    def alloc(n):
        p = vp()
        assert L.sili_buffer_alloc(0, n, C.byref(p)) == 0
        bufs.append(p)
        return p
    try:
        dx, dp, di, dv = alloc(x.nbytes), alloc(12), alloc(12), alloc(12)
        assert L.sili_buffer_copy(0, dx, x.ctypes.data_as(vp), x.nbytes) == 0
        nnz = C.c_int64()
        assert L.sili_dense_to_csr(dx, 2, 3, 0.0, dp, di, dv, 2, C.byref(nnz), None) == 4  # SILI_ERR_RANGE
        assert nnz.value == 3
        assert L.sili_dense_to_csr(dx, 2, 3, 0.0, dp, di, dv, 3, C.byref(nnz), None) == 0
        p = np.zeros(3, np.int32)
        i = np.zeros(3, np.int32)
        assert L.sili_buffer_copy(0, p.ctypes.data_as(vp), dp, 12) == 0
        assert L.sili_buffer_copy(0, i.ctypes.data_as(vp), di, 12) == 0
        assert p.tolist() == [0, 2, 3] and i.tolist() == [0, 2, 1]
    finally:
        for b in bufs:
            L.sili_buffer_free(0, b)
