"""CPU: the built C-ABI library loads and exports every entry point that
include/sili_hip.h declares; argument checks that run before any device call
report SILI_ERR_INVALID.  No compute call is made without a GPU."""
import ctypes as C
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "sili_hip.h")
LIB = os.path.join(ROOT, "sili__new_amd", "libsili_hip.so")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sili_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(LIB):
        pytest.fail("libsili_hip.so is not built (run __graft_entry__.build())")
    return C.CDLL(LIB)


def test_header_declares_the_boundary():
    names = declared()
    for core in ("sili_create", "sili_destroy", "sili_load_weights", "sili_forward_dense",
                 "sili_backward_dense", "sili_sampled_gradw", "sili_forward_sparse",
                 "sili_backward_sparse", "sili_synapto_step", "sili_last_error"):
        assert core in names


def test_every_declared_symbol_is_exported(lib):
    missing = [n for n in declared() if not hasattr(lib, n)]
    assert not missing, missing


def test_create_rejects_bad_shapes_before_touching_a_device(lib):
    lib.sili_create.argtypes = [C.c_int64, C.c_int64, C.c_int64, C.c_int, C.POINTER(C.c_void_p)]
    lib.sili_create.restype = C.c_int
    lib.sili_last_error.restype = C.c_char_p
    h = C.c_void_p()
    for n_in, n_out, mw in ((0, 4, 1), (4, 0, 1), (1 << 31, 4, 1), (4, 4, -1)):
        rc = lib.sili_create(n_in, n_out, mw, 0, C.byref(h))
        assert rc == 1 and not h.value
        assert lib.sili_last_error()
    assert lib.sili_create(4, 4, 1, 0, None) == 1


def test_destroy_null_is_a_no_op(lib):
    lib.sili_destroy.argtypes = [C.c_void_p]
    lib.sili_destroy(None)


def test_pybind_module_imports_and_exports_the_reference_surface():
    """The binding imports without a GPU and carries the reference module's
    names (their GPU behaviour is tested in tests/test_gpu_*)."""
    import sili__new_amd as hip
    for name in ("SparseLinearLayer", "SparseLinearLayerDeterministic", "SparseLinearLayerResync",
                 "SparseLinearLayerResyncDeterministic", "SparseLinearLayerNoScale",
                 "SparseLinearLayerNoScaleDeterministic", "fp4_quantize_array", "dense_to_csr",
                 "dense_to_top_k_csr", "seed_fp4_stochastic_rng"):
        assert hasattr(hip, name), name
