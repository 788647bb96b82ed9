"""ctypes front-end of the CPU oracle (test infrastructure only).

HostLayer holds one layer in the compact host format (numpy arrays) and runs
the restatement's arithmetic on it; RefLayer drives the reference's own
compiled headers through ref_shim.cpp for pinning the restatement.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "liboracle.so"
# The same restatement compiled with a*b+c contracted into FMAs, as the
# reference's own build does: used only to pin the restatement bit-exactly
# against the compiled reference where contraction changes fp32 results.
LIB_FMA_PATH = HERE / "_build" / "liboracle_fma.so"
REF_PATH = HERE / "_ref" / "libsili_ref.so"

_u8p = C.POINTER(C.c_uint8)
_u64p = C.POINTER(C.c_uint64)
_i32p = C.POINTER(C.c_int32)
_f32p = C.POINTER(C.c_float)


def build(ref: bool = True) -> None:
    """Compile the oracle (and, where the reference tree exists, _ref)."""
    targets = ["oracle", "ref"] if ref else ["oracle"]
    subprocess.run(["make", "-s", "-C", str(HERE), *targets], check=True)


class _OracleLayerC(C.Structure):
    _fields_ = [
        ("n_in", C.c_int64), ("n_out", C.c_int64), ("rank", C.c_int32),
        ("row_byte_start", _u64p), ("row_elem_start", _u64p), ("idx", _u8p), ("val", _u8p),
        ("n_tiles", C.c_int64), ("brow_byte_start", _u64p), ("brow_tile_start", _u64p),
        ("bidx", _u8p), ("tiles", _u8p),
        ("value_scale", _f32p), ("output_scale", _f32p),
    ]


class _TrainParams(C.Structure):
    _fields_ = [("lr", C.c_float), ("lr_per_row_nnz", C.c_int32), ("damp_by_importance", C.c_int32),
                ("beta2", C.c_float), ("eps", C.c_float), ("beta1", C.c_float), ("min_decay_frac", C.c_float),
                ("max_abs_delta", C.c_float), ("max_ci", C.c_float), ("zero_escape_eps", C.c_float),
                ("variant", C.c_int32), ("draw_mode", C.c_int32), ("draw_seed", C.c_uint64)]


# the scale-update variants of the reference's layer classes
# (sili/cpu_backend.cpp:992-1013)
TRAIN_VARIANTS = {"plain": 0, "resync": 1, "noscale": 2}


class _B4Merge(C.Structure):
    _fields_ = [("tile_alloc", C.POINTER(C.c_uint64)), ("tile_sparse", C.POINTER(C.c_uint8)),
                ("switch_point", C.c_uint32), ("evicted", C.c_uint64), ("overflow_events", C.c_uint64),
                ("overflow_bytes", C.c_uint64)]


class _B4Res(C.Structure):
    _fields_ = [("ia", C.POINTER(C.c_uint64)), ("ea", C.POINTER(C.c_uint64)), ("ta", C.POINTER(C.c_uint64)),
                ("idx_budget", C.c_uint64), ("tile_budget", C.c_uint64), ("switch_point", C.c_uint32),
                ("flags_in", C.POINTER(C.c_uint8)), ("flags_out", C.POINTER(C.c_uint8)), ("dropped", C.c_uint64)]


class _TrainState(C.Structure):
    _fields_ = [("value_scale", _f32p), ("vs_importance", _f32p), ("vs_momentum", _f32p),
                ("vs_step", C.POINTER(C.c_uint32)), ("output_scale", _f32p), ("os_importance", _f32p),
                ("os_step", C.POINTER(C.c_uint32)), ("importance_scale", _f32p),
                ("output_importance_scale", _f32p), ("out_degree", _i32p), ("output_scale_trainable", C.c_int32),
                ("quant_out", _f32p), ("imp_out", _f32p), ("b4", C.POINTER(_B4Merge))]


# the constants sili/cpu_backend.cpp:496-528 passes to disldo_backward
TRAIN_DEFAULTS = dict(beta1=0.9, min_decay_frac=0.0, max_abs_delta=2.0, max_ci=100.0, zero_escape_eps=0.1)


class _SynStats(C.Structure):
    _fields_ = [(n, C.c_int64) for n in (
        "n_prune_target", "n_pruned", "n_grown", "n_demoted_tiles", "n_promoted_tiles",
        "n_scattered", "n_tiles")]


def _p(a: np.ndarray | None, t):
    if a is None:
        return None
    return a.ctypes.data_as(t)


_libs: dict = {}
_ref = None


def lib(contracted: bool = False):
    """The restatement; contracted=True: its FMA-contracted build."""
    if contracted not in _libs:
        path = LIB_FMA_PATH if contracted else LIB_PATH
        if not path.exists():
            build(ref=False)
        L = C.CDLL(str(path))
        L.oracle_fp4_decode.restype = C.c_float
        L.oracle_fp4_decode.argtypes = [C.c_uint8]
        L.oracle_fp4_encode.restype = C.c_uint8
        L.oracle_fp4_encode.argtypes = [C.c_float]
        L.oracle_fp4_encode_array.argtypes = [_f32p, C.c_int64, _u8p]
        L.oracle_uleb_encode.restype = C.c_size_t
        L.oracle_uleb_encode.argtypes = [C.c_uint32, _u8p]
        L.oracle_csr_index_bytes.restype = C.c_int64
        L.oracle_csr_index_bytes.argtypes = [C.c_int64, _i32p, _i32p]
        L.oracle_csr_encode.argtypes = [C.c_int64, _i32p, _i32p, _f32p, _f32p, _u64p, _u64p, _u8p, _u8p]
        L.oracle_csr_encode_bytes.argtypes = [C.c_int64, _i32p, _i32p, _u8p, _u64p, _u64p, _u8p, _u8p]
        L.oracle_csr_decode.argtypes = [C.c_int64, _u64p, _u64p, _u8p, _i32p]
        L.oracle_combined_to_absolute.restype = C.c_int64
        L.oracle_combined_to_absolute.argtypes = [C.POINTER(_OracleLayerC), _i32p, _i32p, _f32p, _f32p]
        L.oracle_dense_weights.argtypes = [C.POINTER(_OracleLayerC), _f32p]
        L.oracle_forward_dense.argtypes = [C.POINTER(_OracleLayerC), _f32p, C.c_int64, _f32p, C.c_int, C.c_int]
        L.oracle_backward_dense.argtypes = [C.POINTER(_OracleLayerC), _f32p, _f32p, C.c_int64, _f32p,
                                            _f32p, _f32p, C.c_int, C.c_int]
        L.oracle_forward_sparse.argtypes = [C.POINTER(_OracleLayerC), _i32p, _i32p, _f32p, C.c_int64,
                                            _f32p, C.c_int, C.c_int]
        L.oracle_backward_sparse.argtypes = [C.POINTER(_OracleLayerC), _f32p, _i32p, _i32p, _f32p,
                                             C.c_int64, _f32p, _f32p, _f32p, C.c_int, C.c_int]
        L.oracle_sampled_gradw.argtypes = [C.POINTER(_OracleLayerC), _f32p, _f32p, C.c_int64, _f32p,
                                           _f32p, C.c_int, C.c_int]
        L.oracle_backward_train.argtypes = [C.POINTER(_OracleLayerC), _u8p, _u8p, C.POINTER(_TrainState), _f32p, _f32p,
                                            C.c_int64, _f32p, _f32p, _f32p, C.POINTER(_TrainParams)]
        L.oracle_backward_train.restype = C.c_int
        L.oracle_backward_sparse_train.argtypes = [C.POINTER(_OracleLayerC), _u8p, _u8p, C.POINTER(_TrainState), _f32p,
                                                   _i32p, _i32p, _f32p, C.c_int64, _f32p, _f32p, _f32p,
                                                   C.POINTER(_TrainParams)]
        L.oracle_backward_sparse_train.restype = C.c_int
        L.oracle_build_probes.restype = C.c_int64
        L.oracle_build_probes.argtypes = [C.POINTER(_OracleLayerC), _f32p, _f32p, C.c_int64, C.c_int, _i32p, _i32p,
                                          _f32p, C.c_int64]
        L.oracle_synap_row_step.argtypes = [C.POINTER(_OracleLayerC), C.c_int64, _i32p, _i32p, _f32p, C.c_int64,
                                            C.c_int, C.c_float, C.c_int64, C.c_int64, C.c_float, _i32p, _i32p, _i32p,
                                            _u8p, _i32p, _i32p, _u8p, C.POINTER(C.c_int64), _u64p, _u64p,
                                            C.POINTER(C.c_int64)]
        L.oracle_synap_row_step2.argtypes = list(L.oracle_synap_row_step.argtypes) + [C.POINTER(_B4Res)]
        L.oracle_synapto_step.argtypes = [C.POINTER(_OracleLayerC), C.c_float, _i32p, _i32p, _f32p, _f32p,
                                          C.c_int64, C.c_int, _i32p, _i32p, _u8p, _i32p, _i32p, _u8p,
                                          C.POINTER(_SynStats)]
        _libs[contracted] = L
    return _libs[contracted]


def have_ref() -> bool:
    return REF_PATH.exists()


def reflib():
    global _ref
    if _ref is None:
        if not REF_PATH.exists():
            raise FileNotFoundError(f"{REF_PATH} not built (needs the reference tree at build time)")
        R = C.CDLL(str(REF_PATH))
        R.ref_fp4_encode.restype = C.c_uint8
        R.ref_fp4_encode.argtypes = [C.c_float]
        R.ref_fp4_decode.restype = C.c_float
        R.ref_fp4_decode.argtypes = [C.c_uint8]
        R.ref_fp4_table.restype = C.c_float
        R.ref_fp4_table.argtypes = [C.c_uint8]
        R.ref_uleb_encode.restype = C.c_size_t
        R.ref_uleb_encode.argtypes = [C.c_uint32, _u8p]
        R.ref_layer_new.restype = C.c_void_p
        R.ref_layer_new.argtypes = [C.c_int, C.c_int, _i32p, _i32p, _f32p, _f32p]
        R.ref_layer_free.argtypes = [C.c_void_p]
        R.ref_layer_set_scales.argtypes = [C.c_void_p, _f32p, _f32p, C.c_int]
        R.ref_layer_load_dense_codes.argtypes = [C.c_void_p, _u8p, _u8p]
        R.ref_layer_put_tile.argtypes = [C.c_void_p, C.c_int, C.c_int, _u8p]
        R.ref_layer_compact.argtypes = [C.c_void_p]
        R.ref_layer_export.restype = C.c_int64
        R.ref_layer_export.argtypes = [C.c_void_p, _u64p, _u64p, _u8p, _u8p]
        R.ref_layer_nnz_scattered.restype = C.c_int64
        R.ref_layer_nnz_scattered.argtypes = [C.c_void_p]
        R.ref_layer_export_tiles.restype = C.c_int64
        R.ref_layer_export_tiles.argtypes = [C.c_void_p, _i32p, _i32p, _u8p]
        R.ref_layer_combined.restype = C.c_int64
        R.ref_layer_combined.argtypes = [C.c_void_p, _i32p, _i32p, _f32p, _f32p]
        R.ref_forward_dense.argtypes = [C.c_void_p, _f32p, C.c_int, _f32p, C.c_int]
        R.ref_backward_dense.argtypes = [C.c_void_p, _f32p, _f32p, C.c_int, _f32p, _f32p, _f32p, C.c_int]
        R.ref_forward_sparse.argtypes = [C.c_void_p, _i32p, _i32p, _f32p, C.c_int, _f32p, C.c_int]
        R.ref_backward_sparse.argtypes = [C.c_void_p, _f32p, _i32p, _i32p, _f32p, C.c_int, _f32p, _f32p,
                                          _f32p, C.c_int]
        R.ref_row_remove_col.restype = C.c_int
        R.ref_backward_train.argtypes = [C.c_void_p, _f32p, _f32p, C.c_int, _f32p, _f32p, _f32p, C.c_float,
                                         C.c_int, C.c_int, C.c_float, C.c_float, C.c_int, C.c_int]
        R.ref_backward_sparse_train.argtypes = [C.c_void_p, _f32p, _i32p, _i32p, _f32p, C.c_int, _f32p, _f32p, _f32p,
                                                C.c_float, C.c_int, C.c_int, C.c_float, C.c_float, C.c_int]
        R.ref_seed_stochastic.argtypes = [C.c_uint64]
        R.ref_layer_set_importance_scales.argtypes = [C.c_void_p, _f32p, _f32p]
        R.ref_layer_new_blank.restype = C.c_void_p
        R.ref_layer_new_blank.argtypes = [C.c_int, C.c_int, _i32p, _i32p, _f32p, _f32p, C.c_float]
        R.ref_layer_block4_headroom.argtypes = [C.c_void_p, C.c_float, C.c_int]
        R.ref_build_probes.argtypes = [C.c_void_p, _f32p, _f32p, C.c_int, C.c_int]
        R.ref_get_probes.restype = C.c_int64
        R.ref_get_probes.argtypes = [C.c_void_p, _i32p, _i32p, _f32p, C.c_int64, C.POINTER(C.c_int)]
        R.ref_synap_row_step.argtypes = [C.c_void_p, C.POINTER(C.c_int64), C.c_float, C.c_int, C.c_int, C.c_float]
        R.ref_get_out_degree.argtypes = [C.c_void_p, _i32p]
        _u32p = C.POINTER(C.c_uint32)
        R.ref_layer_set_train_state.argtypes = [C.c_void_p, _f32p, _f32p, _u32p, _f32p, _u32p, C.c_int]
        R.ref_layer_get_train_state.argtypes = [C.c_void_p, _f32p, _f32p, _f32p, _u32p, _f32p, _f32p, _u32p]
        R.ref_row_remove_col.argtypes = [C.c_void_p, C.c_int, C.c_int]
        R.ref_row_insert_col.restype = C.c_int
        R.ref_row_insert_col.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_float, C.c_float]
        R.ref_maybe_promote.argtypes = [C.c_void_p, C.c_int, C.c_int]
        R.ref_demote_tile.argtypes = [C.c_void_p, C.c_int, C.c_int]
        R.ref_zero_tile_slot.restype = C.c_int
        R.ref_zero_tile_slot.argtypes = [C.c_void_p, C.c_int, C.c_int]
        R.ref_layer_export_tiles_packed.restype = C.c_int64
        R.ref_layer_export_tiles_packed.argtypes = [C.c_void_p, _u8p, _u8p, _u64p]
        R.ref_block4_switch_point.restype = C.c_uint32
        R.ref_block4_switch_point.argtypes = [C.c_void_p, C.c_int]
        R.ref_block4_used_bytes.restype = C.c_uint64
        R.ref_block4_used_bytes.argtypes = [C.c_void_p]
        R.ref_block4_live.restype = C.c_uint64
        R.ref_block4_live.argtypes = [C.c_void_p]
        R.ref_top_k_csr.restype = C.c_int64
        R.ref_top_k_csr.argtypes = [_f32p, C.c_int, C.c_int, C.c_int, C.c_int, _i32p, _i32p, _f32p]
        R.ref_last_error.restype = C.c_char_p
        R.ref_sll_new.restype = C.c_void_p
        R.ref_sll_new.argtypes = [C.c_int, C.c_int, C.c_int]
        R.ref_sll_load_weights.argtypes = [C.c_void_p, _i32p, _i32p, _f32p, _f32p]
        R.ref_sll_compact.argtypes = [C.c_void_p]
        R.ref_sll_expand.argtypes = [C.c_void_p, C.c_float]
        R.ref_sll_expand_to.argtypes = [C.c_void_p, C.c_int, C.c_float]
        R.ref_sll_equalize_to_capacity.argtypes = [C.c_void_p, C.c_int, C.c_int]
        R.ref_sll_equalizer_step.argtypes = [C.c_void_p]
        R.ref_layer_layout.argtypes = [C.c_void_p, _u64p, _u64p, _u64p, _u64p]
        R.ref_block4_reservations.restype = C.c_int64
        R.ref_block4_reservations.argtypes = [C.c_void_p] + [_u64p] * 7
        R.ref_block4_equalize_step.argtypes = [C.c_void_p]
        R.ref_block4_expand.argtypes = [C.c_void_p, C.c_float, C.c_int]
        R.ref_sll_load_dense_codes.argtypes = [C.c_void_p, _u8p, _u8p]
        R.ref_sll_put_tile.argtypes = [C.c_void_p, C.c_int, C.c_int, _u8p]
        _ref = R
    return _ref


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def _shape2(x):
    x = np.ascontiguousarray(x, np.float32)
    return x.reshape(1, -1) if x.ndim == 1 else x


def dense_to_csr(x, threshold=1e-4):
    """Restatement of the module utility dense_to_csr
    (sili/cpu_backend.cpp:3075-3116): per row, in column order, the entries
    with v > threshold or v < -threshold."""
    x = _shape2(x)
    keep = (x > np.float32(threshold)) | (x < -np.float32(threshold))
    ptrs = np.concatenate([[0], np.cumsum(keep.sum(1))]).astype(np.int32)
    rows, cols = np.nonzero(keep)
    return ptrs, cols.astype(np.int32), x[rows, cols].astype(np.float32)


def dense_to_top_k_csr(x, k):
    """Restatement of dense_to_top_k_csr (csr.hpp:405-505): the min(k, size)
    entries of largest |x| over the flattened array (a global budget), as a
    row-major CSR.  Among equal magnitudes at the cut the lowest flat index
    is kept (the reference leaves that order to its per-thread partial
    sorts, so only cuts between distinct magnitudes are pinned)."""
    x = _shape2(x)
    rows, cols = x.shape
    flat = x.ravel()
    kk = min(int(k), flat.size)
    mag = (flat.view(np.uint32) & np.uint32(0x7FFFFFFF)).astype(np.int64)
    order = np.argsort(-mag, kind="stable")[:kk]
    sel = np.sort(order)
    ptrs = np.searchsorted(sel, np.arange(rows + 1, dtype=np.int64) * cols).astype(np.int32)
    return ptrs, (sel % cols).astype(np.int32), flat[sel].astype(np.float32)


class ScatteredReservations:
    """The reference's per-row reservations of its scattered store
    (DeltaCSRLayout, delta_csr_types.hpp:763-797: byte_start/elem_start with
    blank space between rows) under the calls that set them.  Row contents
    (index bytes, synapses per row) are passed in by the caller; this class
    holds only the reservations b[r], e[r], the budgets and the equalizer
    cursor of SparseLinearLayer (sili/cpu_backend.cpp:371-447, 646-790).

    - from_absolute (delta_csr_memory.hpp:56-66): b = bytes + floor(bytes * f)
      + 5, e = n + max(1, floor(n * f) + 1), the products in fp32;
    - load_weights grows the budgets to the load (:866-876) and reserves with
      f = 0.2; compact (sisldo_ops.hpp:44-96) reserves the content;
    - expand_headroom[_to] (sisldo_ops.hpp:127-186): from_absolute after its
      reserve() calls pass the limits (delta_csr_types.hpp:925-938), sizes in
      double: n' (1 + f) * 6 + 4096 index bytes, (size_t)(n' (1 + f)) + 64
      values, n' = nnz or max(nnz, rows * min_nnz_per_row); MemoryError else;
    - delta_csr_shift_row (delta_csr_memory.hpp:224-293): the byte side, then
      the element side, never on the last row, growth beyond the budget a
      MemoryError (the byte side already moved);
    - equalize_to_capacity (sili/cpu_backend.cpp:684-729), equalizer_step
      (:646-657 -> delta_csr_memory.hpp:295-306)."""

    ULEB_MAX = 5

    def __init__(self, n_in, max_weights):
        self.n = int(n_in)
        self.idx_budget = int(max_weights) * 8 + 4096
        self.val_budget = int(max_weights) + 64
        self.eq = 0
        z = np.zeros(self.n, np.uint64)
        self.from_absolute(z, z, 0.2)

    def from_absolute(self, row_bytes, row_elems, f):
        f = np.float32(f)
        rb = np.asarray(row_bytes, np.uint64)
        re_ = np.asarray(row_elems, np.uint64)
        self.b = rb + (rb.astype(np.float32) * f).astype(np.uint64) + np.uint64(self.ULEB_MAX)
        self.e = re_ + np.maximum(np.uint64(1), (re_.astype(np.float32) * f).astype(np.uint64) + np.uint64(1))
        return self

    def load(self, row_bytes, row_elems):
        nnz = int(np.sum(np.asarray(row_elems, np.uint64)))
        self.idx_budget = max(self.idx_budget, nnz * 8 + 4096)
        self.val_budget = max(self.val_budget, nnz + 64)
        return self.from_absolute(row_bytes, row_elems, 0.2)

    def compact(self, row_bytes, row_elems):
        self.b = np.asarray(row_bytes, np.uint64).copy()
        self.e = np.asarray(row_elems, np.uint64).copy()
        return self

    def expand(self, row_bytes, row_elems, f=0.2, min_nnz_per_row=None):
        n = float(np.sum(np.asarray(row_elems, np.uint64)))
        budget = n if min_nnz_per_row is None else max(n, float(self.n) * float(min_nnz_per_row))
        grow = 1.0 + float(np.float32(f))
        index_bytes = int(budget * grow * (self.ULEB_MAX + 1) + 4096.0)
        values = int(budget * grow) + 64
        if values > self.val_budget or index_bytes > self.idx_budget:
            raise MemoryError("expand_headroom beyond the layer's budget")
        return self.from_absolute(row_bytes, row_elems, f)

    def _shift(self, row, tb, te):
        if row + 1 >= self.n:
            return
        if int(self.b[row]) != tb:
            if tb > int(self.b[row]) and int(self.b.sum()) + tb - int(self.b[row]) > self.idx_budget:
                raise MemoryError("delta_csr_shift_row beyond the layer's budget")
            self.b[row] = tb
        if int(self.e[row]) != te:
            if te > int(self.e[row]) and int(self.e.sum()) + te - int(self.e[row]) > self.val_budget:
                raise MemoryError("delta_csr_shift_row beyond the layer's budget")
            self.e[row] = te

    def equalize_to_capacity(self, te, tb=0):
        te = int(te)
        tb = int(tb) if tb > 0 else te * self.ULEB_MAX + 4
        for r in range(self.n - 1):
            ub, ue = max(int(self.b[r]), tb), max(int(self.e[r]), te)
            if ub == int(self.b[r]) and ue == int(self.e[r]):
                continue
            self._shift(r, ub, ue)
        if self.n > 0:
            self.b[-1] = max(int(self.b[-1]), tb)
            self.e[-1] = max(int(self.e[-1]), te)
        return self

    def equalizer_step(self):
        if self.n == 0:
            return self
        row = self.eq % self.n
        tb = (int(self.b.sum()) + self.n - 1) // self.n
        te = (int(self.e.sum()) + self.n - 1) // self.n
        self._shift(row, tb, te)
        self.eq = (row + 1) % self.n
        return self

    def fit(self, row_bytes, row_elems):
        self.b = np.maximum(self.b, np.asarray(row_bytes, np.uint64))
        self.e = np.maximum(self.e, np.asarray(row_elems, np.uint64))
        return self

    def layout(self, row_bytes, row_elems):
        bs = np.concatenate([[0], np.cumsum(self.b)]).astype(np.uint64)
        es = np.concatenate([[0], np.cumsum(self.e)]).astype(np.uint64)
        return dict(byte_start=bs, byte_end=bs[:-1] + np.asarray(row_bytes, np.uint64),
                    elem_start=es, elem_end=es[:-1] + np.asarray(row_elems, np.uint64))


def row_content(row_byte_start, row_elem_start):
    """(index bytes, synapses) per row of a compact store."""
    return np.diff(np.asarray(row_byte_start, np.uint64)), np.diff(np.asarray(row_elem_start, np.uint64))


def synap_no_room_message(row, fail):
    """delta_csr_synap_row_step's message when an insert does not fit
    (delta_csr_memory.hpp:1239-1248); fail = (probe index, column, used
    bytes, reserved bytes, insertions skipped)."""
    i, col, used, alloc, skipped = (int(v) for v in fail)
    return (f"delta_csr_synap_row_step: row {row} ran out of blank space at probe_index={i} col={col} "
            f"(used {used} / {alloc} bytes, {skipped} insertions skipped). Call equalizer_step() to "
            "redistribute space from adjacent rows before retrying, or reduce max_row_weights / raise "
            "importance_cutoff.")


def demote_no_room_message(fail):
    """block4_demote_tile's message (delta_csr_memory.hpp:985-989)."""
    r, br, bc = (int(v) for v in fail[:3])
    return (f"block4_demote_tile: row {r} ran out of blank space while demoting tile ({br},{bc}). "
            "Call equalizer_step() to redistribute space from adjacent rows before retrying.")


SWITCH_POINT = 10  # BLOCK4_SPARSE_MAX_COUNT (block4.hpp:332-340)


def sparse_pack_tile(tile16):
    """block4_sparse_pack (block4.hpp:364-383), restated: [count] then
    ceil(count/2) bytes of 4-bit slot positions (even index -> high nibble)
    then the count live bytes, slots ascending."""
    t = np.asarray(tile16, np.uint8)
    live = np.flatnonzero(t)
    n = len(live)
    pos = bytearray((n + 1) // 2)
    for i, slot in enumerate(live):
        pos[i // 2] |= (int(slot) << 4) if i % 2 == 0 else int(slot)
    return bytes([n]) + bytes(pos) + bytes(t[live])


def pack_tiles(tiles, flags):
    """A block4 store's tiles as stored bytes: sparse-packed where flags[t],
    else the 16 dense bytes; concatenated in store order."""
    tiles = np.asarray(tiles, np.uint8).reshape(-1, 16)
    out = bytearray()
    for t, f in zip(tiles, flags):
        out += sparse_pack_tile(t) if f else t.tobytes()
    return np.frombuffer(bytes(out), np.uint8).copy()


def tile_live(tiles):
    return (np.asarray(tiles, np.uint8).reshape(-1, 16) != 0).sum(1)


class TileEncodingState:
    """Which block4 tiles the reference stores sparse-packed (tile_is_sparse,
    block4.hpp:1016-1031), restated as the rules its operations apply:

    - a tile written through a handle that was created sparse (every new
      tile: get_or_create starts it sparse-empty, block4.hpp:1150-1183) is
      re-encoded when the handle commits: sparse iff live <= switch_point
      (commit_dirty_sparse_tile, :1226-1290) -- loads (put_tile,
      block4_load_dense, delta_csr_memory.hpp:884-932) and promotion;
    - maybe_compress (:1193-1205), called after promotion and after an
      insert into an existing tile (delta_csr_memory.hpp:656,698), packs a
      dense tile with live <= switch_point;
    - the optimizer updates rewrite every tile they touch through a row
      workspace, re-encoding it by its live count
      (commit_dirty_tile_in_workspace, :1336-1355): the dense update touches
      every tile (linear_disldo.hpp:984-1000: every tiled row counts
      n_tiles * 4 synapses), the sparse-gradient update the tiles with a
      nonzero dy in one of their columns (sisldo_ops.hpp:945-1016);
    - a removal writes the slot to 0 in place: a dense tile stays dense
      (and a tile left with < 2 live slots is demoted away)."""

    def __init__(self, switch_point=SWITCH_POINT):
        self.sp = int(switch_point)
        self.flag = {}

    @staticmethod
    def _keys(br, bc):
        return list(zip(np.asarray(br).tolist(), np.asarray(bc).tolist()))

    def reencode(self, br, bc, tiles, which=None):
        live = tile_live(tiles)
        for i, k in enumerate(self._keys(br, bc)):
            if which is None or which[i]:
                self.flag[k] = int(live[i] <= self.sp)

    load = reencode

    def structural(self, before, after):
        """An edit (removals, inserts into tiles, promotion, demotion) from
        (br, bc, tiles) `before` to `after`."""
        old = {k: t for k, t in zip(self._keys(before[0], before[1]),
                                    np.asarray(before[2], np.uint8).reshape(-1, 16))}
        tiles = np.asarray(after[2], np.uint8).reshape(-1, 16)
        live = tile_live(tiles)
        flag = {}
        for i, k in enumerate(self._keys(after[0], after[1])):
            t = old.get(k)
            if t is None or np.any((t == 0) & (tiles[i] != 0)):
                flag[k] = int(live[i] <= self.sp)  # promoted, or received an insert
            else:
                flag[k] = self.flag[k]
        self.flag = flag

    def flags(self, br, bc):
        return np.array([self.flag[k] for k in self._keys(br, bc)], np.uint8)


def uleb_len(v):
    """Bytes of the unsigned LEB128 encoding of v (delta_csr_types.hpp:209-241)."""
    n = 1
    v = int(v)
    while v >= 0x80:
        v >>= 7
        n += 1
    return n


def tile_len(flag, live):
    """A tile's stored length (block4_stored_tile_len, block4.hpp:340-345,
    386-388): sparse-packed 1 + ceil(live/2) + live, dense 16."""
    live = int(live)
    return 1 + (live + 1) // 2 + live if flag else 16


def tile_len_by_live(live, switch_point=SWITCH_POINT):
    """The length a commit gives a tile: sparse iff live <= switch_point."""
    return tile_len(int(live) <= int(switch_point), live)


class Block4Reservations:
    """The reference's per-block-row reservations of its Block4Store
    (block4.hpp:1016-1031): block-column index bytes ia[br] (block_layout
    byte_start), tile slots ea[br] (elem_start) and tile bytes ta[br]
    (tile_byte_start), the budgets (max_indices_bytes, max_tile_bytes), the
    equalizer cursor and dropped_growth_events, under the calls that set
    them.  Row contents -- used index bytes ui, tiles ue, stored tile bytes
    ut -- are passed in by the caller.

    - the layer's constructor (sili/cpu_backend.cpp:403-441): nothing
      reserved, budgets max_weights*8+4096 and max(4, max_weights/16)*16;
    - block4_row_insert_tile (block4.hpp:670-771): a new tile takes its
      block-column delta change, one slot and 1 tile byte (sparse-empty) of
      its row's room; without room get_or_create (:1170-1183) grows the row
      by block4_ensure_row_headroom (:648-668): +5 index bytes, +1 tile
      byte, +1 slot, through block4_row_shift (:497-617; targets clamped to
      the row's use, index side then tile side then slot side, each growth
      beyond its budget a MemoryError, never on the last row) or
      block4_grow_last_row (:619-646) for the last row;
    - a tile's commit (commit_dirty_sparse_tile, :1226-1290 ->
      block4_resize_tile_in_row, :906-946): growth beyond the row's room
      takes the shortfall from the buffer; beyond max_tile_bytes the commit
      is dropped (dropped_growth_events += 1, the tile keeps its bytes);
    - block4_load_dense (delta_csr_memory.hpp:841-945): new budgets
      (rows*cols*16 index bytes, (size_t)(rows*cols*16 * (1.0 + 0.2f)) +
      rows*16 tile bytes), a tile at every (br, bc) in row-major order,
      each committed, then block4_expand_headroom(0.2);
    - block4_expand_headroom (:767-823): ta = ut + (size_t)(ut * f) + slack,
      the product in fp32, MemoryError beyond max_tile_bytes (nothing
      changed); compact_block4 is f = 0, slack 0;
    - Block4Store::equalize_step (block4.hpp:1208-1220): the cursor row
      shifted towards the ceil-average of each reservation."""

    ULEB_MAX = 5
    NO_LIMIT = (1 << 64) - 1

    def __init__(self, n_in, max_weights=None, switch_point=SWITCH_POINT):
        self.rows = (int(n_in) + 3) // 4
        self.ia = [0] * self.rows
        self.ea = [0] * self.rows
        self.ta = [0] * self.rows
        if max_weights is None:
            self.idx_budget = self.tile_budget = self.NO_LIMIT
        else:
            self.idx_budget = int(max_weights) * 8 + 4096
            self.tile_budget = max(4, int(max_weights) // 16) * 16
        self.sp = int(switch_point)
        self.eq = 0
        self.dropped = 0

    # -- block4_row_shift / block4_grow_last_row / ensure_row_headroom --------
    def _shift(self, row, ti, tt, te, ui, ue, ut):
        ti, tt, te = max(ti, ui), max(tt, ut), max(te, ue)
        if row + 1 >= self.rows:
            return
        if self.ia[row] != ti:
            if ti > self.ia[row] and sum(self.ia) + ti - self.ia[row] > self.idx_budget:
                raise MemoryError("block4_row_shift: index bytes beyond max_indices_bytes")
            self.ia[row] = ti
        if self.ta[row] != tt:
            if tt > self.ta[row] and sum(self.ta) + tt - self.ta[row] > self.tile_budget:
                raise MemoryError("block4_row_shift: tile bytes beyond max_tile_bytes")
            self.ta[row] = tt
        if self.ea[row] != te:
            self.ea[row] = te

    def _grow_last(self, ti, tt, te):
        r = self.rows - 1
        if ti > self.ia[r]:
            if sum(self.ia) + ti - self.ia[r] > self.idx_budget:
                raise MemoryError("block4_grow_last_row: index bytes beyond max_indices_bytes")
            self.ia[r] = ti
        if tt > self.ta[r]:
            if sum(self.ta) + tt - self.ta[r] > self.tile_budget:
                raise MemoryError("block4_grow_last_row: tile bytes beyond max_tile_bytes")
            self.ta[r] = tt
        if te > self.ea[r]:
            self.ea[r] = te

    def insert_tile(self, row, idx_delta, ui, ue, ut):
        """get_or_create of a new tile in block row `row` whose block-column
        delta bytes change by idx_delta; (ui, ue, ut) is the row's use
        before.  Returns the use after (the new tile sparse-empty, 1 byte)."""
        fits = (not (idx_delta > 0 and idx_delta > self.ia[row] - ui) and ue < self.ea[row]
                and 1 <= self.ta[row] - ut)
        if not fits:
            ti, tt, te = self.ia[row] + self.ULEB_MAX, self.ta[row] + 1, self.ea[row] + 1
            if row + 1 < self.rows:
                self._shift(row, ti, tt, te, ui, ue, ut)
            else:
                self._grow_last(ti, tt, te)
        return ui + idx_delta, ue + 1, ut + 1

    def commit(self, row, old_len, new_len, ut):
        """A tile of block row `row` re-stored from old_len to new_len bytes;
        ut: the row's stored bytes before.  Returns (committed, ut after)."""
        d = int(new_len) - int(old_len)
        if d > 0:
            room = self.ta[row] - ut
            if d > room:
                short = d - room
                if sum(self.ta) + short > self.tile_budget:
                    self.dropped += 1
                    return False, ut
                self.ta[row] += short
        return True, ut + d

    # -- whole-store calls -------------------------------------------------------
    def load_dense(self, n_in, n_out, wc, ic):
        """block4_load_dense of codes wc, ic [n_in * n_out]; returns the use
        (ui, ue, ut) per block row."""
        brows, bcols = (n_in + 3) // 4, (n_out + 3) // 4
        assert brows == self.rows
        self.ia, self.ea, self.ta = [0] * brows, [0] * brows, [0] * brows
        self.idx_budget = brows * bcols * 16
        self.tile_budget = int(float(brows * bcols * 16) * (1.0 + float(np.float32(0.2)))) + brows * 16
        codes = np.zeros((brows * 4, bcols * 4), np.uint8)
        codes[:n_in, :n_out] = (np.asarray(wc, np.uint8) | (np.asarray(ic, np.uint8) << 4)).reshape(n_in, n_out)
        live = (codes.reshape(brows, 4, bcols, 4) != 0).sum(axis=(1, 3))
        ui, ue, ut = [0] * brows, [0] * brows, [0] * brows
        for br in range(brows):
            u = (0, 0, 0)
            for bc in range(bcols):
                u = self.insert_tile(br, 1, *u)  # deltas 0, 1, 1, ...: one byte each
                ok, t = self.commit(br, 1, tile_len_by_live(live[br, bc], self.sp), u[2])
                u = (u[0], u[1], t)
            ui[br], ue[br], ut[br] = u
        self.expand(ut, 0.2, 16)
        return ui, ue, ut

    def expand(self, ut, f=0.2, slack=16):
        f = np.float32(f)
        new = [int(u) + int(np.float32(u) * f) + int(slack) for u in ut]
        if sum(new) > self.tile_budget:
            raise MemoryError("block4_expand_headroom beyond max_tile_bytes")
        self.ta = new
        return self

    def compact(self, ut):
        return self.expand(ut, 0.0, 0)

    def equalize_step(self, ui, ue, ut):
        if self.rows == 0:
            return self
        row = self.eq % self.rows
        n = self.rows
        ti = (sum(self.ia) + n - 1) // n
        tt = (sum(self.ta) + n - 1) // n
        te = (sum(self.ea) + n - 1) // n
        self._shift(row, ti, tt, te, int(ui[row]), int(ue[row]), int(ut[row]))
        self.eq = (self.eq + 1) % n
        return self


def block4_row_use(n_in, br, bc, tiles, flags):
    """(ui, ue, ut) per block row of a compact block4 store (tiles sorted by
    (br, bc)): block-column ULEB128 bytes, tiles, stored tile bytes."""
    rows = (int(n_in) + 3) // 4
    ui, ue, ut = [0] * rows, [0] * rows, [0] * rows
    live = tile_live(tiles)
    prev_r, prev_c = -1, 0
    for i, (r, c) in enumerate(zip(np.asarray(br).tolist(), np.asarray(bc).tolist())):
        if r != prev_r:
            prev_r, prev_c = r, 0
        ui[r] += uleb_len(c - prev_c)
        prev_c = c
        ue[r] += 1
        ut[r] += tile_len(flags[i], live[i])
    return ui, ue, ut


class Block4PutModel:
    """A block4 store's tiles as Block4Store::get_or_create and a handle's
    slot writes leave them (block4.hpp:1170-1183,1226-1290; the reference's
    own tests' fixture, test_disldo_block4_forward.cpp:34-45), with their
    tile_is_sparse flags and the store's reservations (Block4Reservations)
    alongside.  put() raises MemoryError where get_or_create's row growth
    meets a budget; a commit dropped at the tile budget leaves the tile as
    it was."""

    def __init__(self, n_in, max_weights):
        self.n_in = n_in
        self.M = Block4Reservations(n_in, max_weights)
        self.sp = self.M.sp
        self.rows = [dict() for _ in range(self.M.rows)]  # bc -> (flag, 16 bytes)

    def use(self):
        ui, ue, ut = [], [], []
        for row in self.rows:
            cols = sorted(row)
            ui.append(sum(uleb_len(c - p) for c, p in zip(cols, [0] + cols[:-1])))
            ue.append(len(cols))
            ut.append(sum(tile_len(row[c][0], np.count_nonzero(row[c][1])) for c in cols))
        return ui, ue, ut

    def put(self, br, bc, tile):
        row = self.rows[br]
        ui, ue, ut = (u[br] for u in self.use())
        if bc not in row:
            cols = sorted(row)
            prev = max([c for c in cols if c < bc], default=0)
            nxt = min([c for c in cols if c > bc], default=None)
            d = uleb_len(bc - prev)
            if nxt is not None:
                d += uleb_len(nxt - bc) - uleb_len(nxt - prev)
            self.M.insert_tile(br, d, ui, ue, ut)  # raises MemoryError with the row unchanged
            row[bc] = (1, np.zeros(16, np.uint8))
            ut += 1
        flag, old = row[bc]
        if flag:  # a sparse tile's handle writes a scratch copy and commits it
            ok, _ = self.M.commit(br, tile_len(1, np.count_nonzero(old)), tile_len_by_live(np.count_nonzero(tile), self.sp), ut)
            if ok:
                row[bc] = (int(np.count_nonzero(tile) <= self.sp), tile.copy())
        else:  # a dense tile is written in place
            row[bc] = (0, tile.copy())


    def canonical(self):
        """(br, bc, tiles, flags) in canonical order."""
        keys = [(b, c) for b, row in enumerate(self.rows) for c in sorted(row)]
        br = np.array([k[0] for k in keys], np.int32)
        bc = np.array([k[1] for k in keys], np.int32)
        tiles = np.concatenate([self.rows[b][c][1] for b, c in keys]) if keys else np.zeros(0, np.uint8)
        flags = np.array([self.rows[b][c][0] for b, c in keys], np.uint8)
        return br, bc, tiles, flags


def block4_put_layer(n_in, max_weights, br, bc, tiles):
    """The store a layer's tiles placed one by one in canonical order leave
    (load_block4_tiles): (Block4PutModel, flags in canonical order)."""
    T = Block4PutModel(n_in, max_weights)
    tiles = np.asarray(tiles, np.uint8).reshape(-1, 16)
    for i in np.lexsort((np.asarray(bc), np.asarray(br))):
        T.put(int(br[i]), int(bc[i]), tiles[i])
    return T, T.canonical()[3]


FOR_REF_PATH = HERE / "_ref" / "libfor_ref.so"
_for_ref = None


def for_encode_row(cols, G=16):
    """Restatement of the reference prototype's group frame-of-reference
    encoder (prototypes/for_delta_encoding/for_encoding_bench.cpp:31-54,
    README.md:18-40) for one row's sorted columns: groups of G values, each
    a tier byte (0/1/2: 1/2/4 bytes per offset, by the group's largest
    offset) then G little-endian offsets from the group start (the previous
    group's last column, 0 for the first); a short last group repeats its
    last offset."""
    cols = np.asarray(cols, np.int64)
    out = bytearray()
    start = 0
    for g0 in range(0, len(cols), G):
        grp = cols[g0:g0 + G]
        off = np.full(G, grp[-1] - start, np.int64)
        off[:len(grp)] = grp - start
        m = int(off[-1])
        tier = 0 if m < 256 else (1 if m < 65536 else 2)
        w = (1, 2, 4)[tier]
        out.append(tier)
        out += off.astype({1: "<u1", 2: "<u2", 4: "<u4"}[w]).tobytes()
        start = int(grp[-1])
    return bytes(out)


def for_encode_rows(ptrs, cols, G=16):
    """FOR bytes of every row, concatenated; returns (row_byte_start, bytes)."""
    ptrs = np.asarray(ptrs, np.int64)
    parts, starts, n = [], [0], 0
    for r in range(len(ptrs) - 1):
        b = for_encode_row(cols[ptrs[r]:ptrs[r + 1]], G)
        parts.append(b)
        n += len(b)
        starts.append(n)
    return np.array(starts, np.uint64), np.frombuffer(b"".join(parts), np.uint8).copy()


def ref_for_encode(cols, G=16):
    """The reference prototype's own encoder (compiled from its source, _ref)
    on one row's columns."""
    global _for_ref
    if _for_ref is None:
        R = C.CDLL(str(FOR_REF_PATH))
        R.ref_for_encode.restype = C.c_int64
        R.ref_for_encode.argtypes = [C.POINTER(C.c_uint32), C.c_int64, C.c_int, _u8p, C.c_int64]
        _for_ref = R
    cols = np.asarray(cols, np.int64)
    d = np.diff(np.concatenate([[0], cols])).astype(np.uint32)
    cap = 1 + (len(d) // G + 1) * (1 + 4 * G)
    out = np.zeros(cap, np.uint8)
    n = _for_ref.ref_for_encode(d.ctypes.data_as(C.POINTER(C.c_uint32)), len(d), int(G), _p(out, _u8p), cap)
    assert n >= 0
    return out[:n].tobytes()


def ref_top_k_csr(x, k, threads=4):
    """The reference's own top_k_csr (compiled from its header, _ref)."""
    x = _shape2(x).copy()
    rows, cols = x.shape
    kk = min(int(k), x.size)
    ptrs = np.zeros(rows + 1, np.int32)
    idx = np.zeros(max(kk, 1), np.int32)
    vals = np.zeros(max(kk, 1), np.float32)
    n = reflib().ref_top_k_csr(_p(x, _f32p), rows, cols, int(k), int(threads), _p(ptrs, _i32p), _p(idx, _i32p),
                               _p(vals, _f32p))
    return ptrs, idx[:n], vals[:n]


def encode_tiles(n_in: int, br: np.ndarray, bc: np.ndarray, tiles: np.ndarray):
    """Block4 store (block-row CSR, ULEB block-column deltas) from a tile
    list; returns (brow_byte_start, brow_tile_start, bidx, tiles sorted)."""
    br = np.asarray(br, np.int64)
    bc = np.asarray(bc, np.int64)
    order = np.lexsort((bc, br))
    br, bc = br[order], bc[order]
    t = np.ascontiguousarray(np.asarray(tiles, np.uint8).reshape(-1, 16)[order]).ravel()
    brows = (n_in + 3) // 4
    ptrs = np.zeros(brows + 1, np.int32)
    np.add.at(ptrs, br + 1, 1)
    ptrs = np.cumsum(ptrs).astype(np.int32)
    L = lib()
    nb = L.oracle_csr_index_bytes(brows, _p(ptrs, _i32p), _p(_c(bc, np.int32), _i32p))
    bs = np.zeros(brows + 1, np.uint64)
    ts = np.zeros(brows + 1, np.uint64)
    idx = np.zeros(max(1, nb), np.uint8)
    dummy = np.zeros(max(1, len(bc)), np.uint8)
    rc = L.oracle_csr_encode_bytes(brows, _p(ptrs, _i32p), _p(_c(bc, np.int32), _i32p), _p(dummy, _u8p),
                                   _p(bs, _u64p), _p(ts, _u64p), _p(idx, _u8p), _p(dummy.copy(), _u8p))
    if rc != 0:
        raise ValueError("tile list has duplicates")
    return bs, ts, idx[:nb], t, br.astype(np.int32), bc.astype(np.int32)


class HostLayer:
    """A layer in the compact host format, evaluated by the CPU restatement."""

    def __init__(self, n_in: int, n_out: int, rank: int = 1):
        self.n_in, self.n_out, self.rank = int(n_in), int(n_out), int(rank)
        self.row_byte_start = np.zeros(n_in + 1, np.uint64)
        self.row_elem_start = np.zeros(n_in + 1, np.uint64)
        self.idx = np.zeros(1, np.uint8)
        self.val = np.zeros(1, np.uint8)
        self.nnz = 0
        self.index_bytes = 0
        self.n_tiles = 0
        self.brow_byte_start = np.zeros((n_in + 3) // 4 + 1, np.uint64)
        self.brow_tile_start = np.zeros((n_in + 3) // 4 + 1, np.uint64)
        self.bidx = np.zeros(1, np.uint8)
        self.tiles = np.zeros(16, np.uint8)
        self.tile_br = np.zeros(0, np.int32)
        self.tile_bc = np.zeros(0, np.int32)
        vs = np.zeros(n_in * rank, np.float32)
        vs[::rank] = 1.0
        os_ = np.zeros(n_out * rank, np.float32)
        os_[::rank] = 1.0
        self.value_scale, self.output_scale = vs, os_
        # the scales' optimizer state (delta_csr_types.hpp:1127-1215)
        self.vs_importance = np.zeros(n_in * rank, np.float32)
        self.vs_momentum = np.zeros(n_in * rank, np.float32)
        self.vs_step = np.zeros(n_in * rank, np.uint32)
        self.os_importance = np.zeros(n_out * rank, np.float32)
        self.os_step = np.zeros(n_out * rank, np.uint32)
        self.importance_scale = None
        self.output_importance_scale = None
        self.output_scale_trainable = False
        # the block rows' tile-byte reservations and the tiles' encoding, for
        # the updates' write-back (None: rows taken to have room)
        self.b4_alloc = None   # uint64 [ceil(n_in/4)]
        self.b4_flags = None   # uint8 [n_tiles], tile_is_sparse in canonical order
        self.b4res = None      # a Block4Reservations: the policy keeps it, the updates read its ta
        self.b4_switch_point = SWITCH_POINT
        self.b4_counters = [0, 0, 0]  # evicted slots, merge overflow events, overflow bytes

    # -- construction ----------------------------------------------------------
    def load_csr(self, ptrs, cols, w=None, imp=None, bytes_=None):
        ptrs = _c(ptrs, np.int32)
        cols = _c(cols, np.int32)
        L = lib()
        nb = L.oracle_csr_index_bytes(self.n_in, _p(ptrs, _i32p), _p(cols, _i32p))
        self.idx = np.zeros(max(1, nb), np.uint8)
        self.val = np.zeros(max(1, len(cols)), np.uint8)
        if bytes_ is not None:
            rc = L.oracle_csr_encode_bytes(self.n_in, _p(ptrs, _i32p), _p(cols, _i32p),
                                           _p(_c(bytes_, np.uint8), _u8p), _p(self.row_byte_start, _u64p),
                                           _p(self.row_elem_start, _u64p), _p(self.idx, _u8p),
                                           _p(self.val, _u8p))
        else:
            wv = _c(w, np.float32)
            iv = None if imp is None else _c(imp, np.float32)
            rc = L.oracle_csr_encode(self.n_in, _p(ptrs, _i32p), _p(cols, _i32p), _p(wv, _f32p),
                                     _p(iv, _f32p), _p(self.row_byte_start, _u64p),
                                     _p(self.row_elem_start, _u64p), _p(self.idx, _u8p), _p(self.val, _u8p))
        if rc != 0:
            raise ValueError("columns must be strictly increasing within a row")
        self.nnz = len(cols)
        self.index_bytes = nb
        return self

    def load_encoded(self, row_byte_start, row_elem_start, idx, val):
        """Take an already encoded scattered store (e.g. a device export)."""
        self.row_byte_start = _c(row_byte_start, np.uint64).copy()
        self.row_elem_start = _c(row_elem_start, np.uint64).copy()
        self.index_bytes = int(self.row_byte_start[-1])
        self.nnz = int(self.row_elem_start[-1])
        self.idx = np.concatenate([_c(idx, np.uint8), np.zeros(8, np.uint8)])
        self.val = np.concatenate([_c(val, np.uint8), np.zeros(8, np.uint8)])
        return self

    def load_tiles(self, br, bc, tiles):
        (self.brow_byte_start, self.brow_tile_start, self.bidx, self.tiles,
         self.tile_br, self.tile_bc) = encode_tiles(self.n_in, br, bc, tiles)
        self.n_tiles = len(self.tile_br)
        if self.n_tiles == 0:
            self.tiles = np.zeros(16, np.uint8)
        if len(self.bidx) == 0:
            self.bidx = np.zeros(1, np.uint8)
        return self

    def set_scales(self, vs=None, os_=None):
        if vs is not None:
            self.value_scale = _c(vs, np.float32).copy()
        if os_ is not None:
            self.output_scale = _c(os_, np.float32).copy()
        return self

    def _cstruct(self) -> _OracleLayerC:
        s = _OracleLayerC()
        s.n_in, s.n_out, s.rank = self.n_in, self.n_out, self.rank
        s.row_byte_start = _p(self.row_byte_start, _u64p)
        s.row_elem_start = _p(self.row_elem_start, _u64p)
        s.idx, s.val = _p(self.idx, _u8p), _p(self.val, _u8p)
        s.n_tiles = self.n_tiles
        s.brow_byte_start = _p(self.brow_byte_start, _u64p)
        s.brow_tile_start = _p(self.brow_tile_start, _u64p)
        s.bidx, s.tiles = _p(self.bidx, _u8p), _p(self.tiles, _u8p)
        s.value_scale, s.output_scale = _p(self.value_scale, _f32p), _p(self.output_scale, _f32p)
        return s

    # -- structure ---------------------------------------------------------------
    def decode_cols(self) -> np.ndarray:
        n = int(self.row_elem_start[-1])
        out = np.zeros(max(1, n), np.int32)
        if lib().oracle_csr_decode(self.n_in, _p(self.row_byte_start, _u64p), _p(self.row_elem_start, _u64p),
                                   _p(self.idx, _u8p), _p(out, _i32p)) != 0:
            raise ValueError("index stream does not match its row ends")
        return out[:n]

    def absolute(self):
        s = self._cstruct()
        n = lib().oracle_combined_to_absolute(C.byref(s), None, None, None, None)
        p = np.zeros(self.n_in + 1, np.int32)
        ix = np.zeros(max(1, n), np.int32)
        w = np.zeros(max(1, n), np.float32)
        imp = np.zeros(max(1, n), np.float32)
        lib().oracle_combined_to_absolute(C.byref(s), _p(p, _i32p), _p(ix, _i32p), _p(w, _f32p), _p(imp, _f32p))
        return p, ix[:n], w[:n], imp[:n]

    def dense(self) -> np.ndarray:
        W = np.zeros((self.n_in, self.n_out), np.float32)
        s = self._cstruct()
        lib().oracle_dense_weights(C.byref(s), _p(W, _f32p))
        return W

    # -- compute (fresh outputs) ---------------------------------------------------
    def forward_dense(self, x, threads=8, absmode=False):
        x = _c(np.atleast_2d(x), np.float32)
        y = np.zeros((x.shape[0], self.n_out), np.float32)
        s = self._cstruct()
        lib().oracle_forward_dense(C.byref(s), _p(x, _f32p), x.shape[0], _p(y, _f32p), threads, int(absmode))
        return y

    def backward_dense(self, x, dy, threads=8, absmode=False, acc=None):
        x = _c(np.atleast_2d(x), np.float32)
        dy = _c(np.atleast_2d(dy), np.float32)
        dx = np.zeros_like(x)
        ai = np.zeros(self.n_in, np.float32) if acc is None else acc[0]
        ag = np.zeros(self.n_out, np.float32) if acc is None else acc[1]
        s = self._cstruct()
        lib().oracle_backward_dense(C.byref(s), _p(x, _f32p), _p(dy, _f32p), x.shape[0], _p(dx, _f32p),
                                    _p(ai, _f32p), _p(ag, _f32p), threads, int(absmode))
        return dx, ai, ag

    def forward_sparse(self, ptrs, idx, vals, batch, threads=8, absmode=False):
        ptrs, idx, vals = _c(ptrs, np.int32), _c(idx, np.int32), _c(vals, np.float32)
        y = np.zeros((batch, self.n_out), np.float32)
        s = self._cstruct()
        lib().oracle_forward_sparse(C.byref(s), _p(ptrs, _i32p), _p(idx, _i32p), _p(vals, _f32p), batch,
                                    _p(y, _f32p), threads, int(absmode))
        return y

    def backward_sparse(self, x, dptrs, didx, dvals, batch, threads=8, absmode=False):
        x = _c(np.atleast_2d(x), np.float32)
        dptrs, didx, dvals = _c(dptrs, np.int32), _c(didx, np.int32), _c(dvals, np.float32)
        dx = np.zeros_like(x)
        ai = np.zeros(self.n_in, np.float32)
        ag = np.zeros(self.n_out, np.float32)
        s = self._cstruct()
        lib().oracle_backward_sparse(C.byref(s), _p(x, _f32p), _p(dptrs, _i32p), _p(didx, _i32p),
                                     _p(dvals, _f32p), batch, _p(dx, _f32p), _p(ai, _f32p), _p(ag, _f32p),
                                     threads, int(absmode))
        return dx, ai, ag

    def out_degree(self) -> np.ndarray:
        return np.bincount(self.decode_cols(), minlength=self.n_out).astype(np.int32)

    def _b4_merge(self):
        alloc = self.b4res.ta if self.b4res is not None else self.b4_alloc
        if alloc is None or self.n_tiles == 0:
            return None
        self._b4_alloc_c = np.ascontiguousarray(np.asarray(alloc, np.uint64))
        assert len(self.b4_flags) >= self.n_tiles
        return _B4Merge(self._b4_alloc_c.ctypes.data_as(C.POINTER(C.c_uint64)),
                        self.b4_flags.ctypes.data_as(C.POINTER(C.c_uint8)), int(self.b4_switch_point), 0, 0, 0)

    def _b4_merged(self, m):
        if m is not None:
            self.b4_counters = [self.b4_counters[0] + m.evicted, self.b4_counters[1] + m.overflow_events,
                                self.b4_counters[2] + m.overflow_bytes]

    def backward_train(self, x, dy, lr, lr_per_row_nnz=False, damp_by_importance=True, beta2=0.999, eps=1e-8,
                       acc=None, contracted=False, variant="plain"):
        """Backward with the optimizer update (deterministic rounding, one
        thread): updates self.val and the scale state in place; returns dx and
        the activity accumulators.  self.last_quant / self.last_imp: every
        synapse's weight code value and importance before re-quantization.
        contracted=True runs the FMA-contracted build of the restatement.
        variant: "plain", "resync" (DeferredScaleWrite) or "noscale"."""
        self.last_quant = np.zeros(max(1, self.nnz), np.float32)
        self.last_imp = np.zeros(max(1, self.nnz), np.float32)
        x = _c(np.atleast_2d(x), np.float32)
        dy = _c(np.atleast_2d(dy), np.float32)
        dx = np.zeros_like(x)
        ai = np.zeros(self.n_in, np.float32) if acc is None else acc[0]
        ag = np.zeros(self.n_out, np.float32) if acc is None else acc[1]
        deg = self.out_deg if getattr(self, "out_deg", None) is not None else self.out_degree()
        isc = None if self.importance_scale is None else _c(self.importance_scale, np.float32)
        oisc = None if self.output_importance_scale is None else _c(self.output_importance_scale, np.float32)
        u32p = C.POINTER(C.c_uint32)
        m = self._b4_merge()
        st = _TrainState(_p(self.value_scale, _f32p), _p(self.vs_importance, _f32p), _p(self.vs_momentum, _f32p),
                         _p(self.vs_step, u32p), _p(self.output_scale, _f32p), _p(self.os_importance, _f32p),
                         _p(self.os_step, u32p), _p(isc, _f32p), _p(oisc, _f32p), _p(deg, _i32p),
                         int(self.output_scale_trainable), _p(self.last_quant, _f32p), _p(self.last_imp, _f32p),
                         None if m is None else C.pointer(m))
        P = _TrainParams(lr, int(lr_per_row_nnz), int(damp_by_importance), beta2, eps, **TRAIN_DEFAULTS,
                         variant=TRAIN_VARIANTS[variant])
        s = self._cstruct()
        tiles = self.tiles.copy() if self.n_tiles > 0 else None
        if lib(contracted).oracle_backward_train(C.byref(s), _p(self.val, _u8p), _p(tiles, _u8p), C.byref(st),
                                                 _p(x, _f32p), _p(dy, _f32p), x.shape[0], _p(dx, _f32p),
                                                 _p(ai, _f32p), _p(ag, _f32p), C.byref(P)) != 0:
            raise ValueError("backward_train failed")
        if tiles is not None:
            self.tiles[:] = tiles
        self._b4_merged(m)
        return dx, ai, ag

    def backward_sparse_train(self, x, dptrs, didx, dvals, batch, lr, lr_per_row_nnz=False, damp_by_importance=True,
                              beta2=0.999, eps=1e-8, contracted=False, draw_mode=1, draw_seed=0):
        """backward_sparse with the optimizer update (one thread): updates
        self.val, self.tiles and the value scales' state in place; returns dx
        and the activity accumulators.  draw_mode / draw_seed: the block4
        tiles' stochastic rounding (0: the reference's seeded per-thread
        xorshift64*, 1: the GPU library's counter draws)."""
        x = _c(np.atleast_2d(x), np.float32)
        dptrs, didx, dvals = _c(dptrs, np.int32), _c(didx, np.int32), _c(dvals, np.float32)
        dx = np.zeros_like(x)
        ai = np.zeros(self.n_in, np.float32)
        ag = np.zeros(self.n_out, np.float32)
        isc = None if self.importance_scale is None else _c(self.importance_scale, np.float32)
        oisc = None if self.output_importance_scale is None else _c(self.output_importance_scale, np.float32)
        u32p = C.POINTER(C.c_uint32)
        m = self._b4_merge()
        st = _TrainState(_p(self.value_scale, _f32p), _p(self.vs_importance, _f32p), _p(self.vs_momentum, _f32p),
                         _p(self.vs_step, u32p), _p(self.output_scale, _f32p), _p(self.os_importance, _f32p),
                         _p(self.os_step, u32p), _p(isc, _f32p), _p(oisc, _f32p), None, 0, None, None,
                         None if m is None else C.pointer(m))
        P = _TrainParams(lr, int(lr_per_row_nnz), int(damp_by_importance), beta2, eps, **TRAIN_DEFAULTS, variant=0,
                         draw_mode=int(draw_mode), draw_seed=int(draw_seed) & (2**64 - 1))
        s = self._cstruct()
        tiles = _p(self.tiles, _u8p) if self.n_tiles > 0 else None
        if lib(contracted).oracle_backward_sparse_train(C.byref(s), _p(self.val, _u8p), tiles, C.byref(st), _p(x, _f32p),
                                                        _p(dptrs, _i32p), _p(didx, _i32p), _p(dvals, _f32p), batch,
                                                        _p(dx, _f32p), _p(ai, _f32p), _p(ag, _f32p),
                                                        C.byref(P)) != 0:
            raise ValueError("backward_sparse_train: tile bytes missing")
        self._b4_merged(m)
        return dx, ai, ag

    # -- the reference's synaptogenesis policy (delta_csr_memory.hpp:1021-1426) --
    def build_probes(self, acc_in, acc_grad, k, per_row=False):
        """delta_csr_build_probes with the given activity accumulators."""
        acc_in, acc_grad = _c(acc_in, np.float32), _c(acc_grad, np.float32)
        kk = max(int(k), 0)
        cap = max(1, kk * kk if not per_row else kk * max(kk, 1)) + 1
        cap = max(cap, kk * min(kk, self.n_out) + 1)
        prow, pcol = np.zeros(cap, np.int32), np.zeros(cap, np.int32)
        pval = np.zeros(cap, np.float32)
        s = self._cstruct()
        n = lib().oracle_build_probes(C.byref(s), _p(acc_in, _f32p), _p(acc_grad, _f32p), int(k), int(per_row),
                                      _p(prow, _i32p), _p(pcol, _i32p), _p(pval, _f32p), cap)
        if not hasattr(self, "probes"):
            self.probes = (np.zeros(0, np.int32), np.zeros(0, np.int32), np.zeros(0, np.float32))
            self.probe_nnz = 0
        if n < 0:               # the reference zeroes the count, keeps the old vectors
            self.probe_nnz = 0
            return
        assert n <= cap
        self.probes = (prow[:n].copy(), pcol[:n].copy(), pval[:n].copy())
        self.probe_nnz = int(n)

    def synap_row_step(self, current_row, importance_cutoff, max_row_weights, max_prune_per_step=8,
                       importance_eps=1e-3, reservations=None):
        """delta_csr_synap_row_step: returns (did, next cursor).  With
        reservations (a ScatteredReservations), an insert or a demotion that
        does not fit raises RuntimeError with the reference's message: the
        removals and earlier inserts stay applied after an insert's failure,
        nothing does after a demotion's."""
        if self.n_in == 0:
            return False, current_row
        row = int(current_row) % self.n_in
        nxt = (int(current_row) + 1) % self.n_in
        if not hasattr(self, "probes"):
            self.probes = (np.zeros(0, np.int32), np.zeros(0, np.int32), np.zeros(0, np.float32))
            self.probe_nnz = 0
        if getattr(self, "out_deg", None) is None:
            self.out_deg = self.out_degree().astype(np.int32)
        prow, pcol, pval = (_c(a, t) for a, t in zip(self.probes, (np.int32, np.int32, np.float32)))
        nnz, nt = self.nnz, self.n_tiles
        cap_s = nnz + len(prow) + 16 * nt + 1
        cap_t = nt + len(prow) + 1
        ptrs = np.zeros(self.n_in + 1, np.int32)
        cols = np.zeros(cap_s, np.int32)
        byts = np.zeros(cap_s, np.uint8)
        tbr, tbc = np.zeros(cap_t, np.int32), np.zeros(cap_t, np.int32)
        tby = np.zeros(16 * cap_t, np.uint8)
        ntl = C.c_int64(0)
        s = self._cstruct()
        rb = re_ = None
        if reservations is not None:
            rb = _c(reservations.b, np.uint64)
            re_ = _c(reservations.e, np.uint64)
        fail = np.zeros(5, np.int64)
        b4 = None
        if self.b4res is not None:
            R = self.b4res
            arrs = [np.array(v, np.uint64) for v in (R.ia, R.ea, R.ta)]
            fin = np.ascontiguousarray(self.b4_flags[:max(1, nt)], np.uint8)
            fout = np.zeros(cap_t, np.uint8)
            u64p = C.POINTER(C.c_uint64)
            b4 = _B4Res(*[a.ctypes.data_as(u64p) for a in arrs], R.idx_budget, R.tile_budget, R.sp,
                        fin.ctypes.data_as(C.POINTER(C.c_uint8)), fout.ctypes.data_as(C.POINTER(C.c_uint8)),
                        R.dropped)
        did = lib().oracle_synap_row_step2(C.byref(s), row, _p(prow, _i32p), _p(pcol, _i32p), _p(pval, _f32p),
                                           self.probe_nnz, int(len(prow) > 0), importance_cutoff,
                                           int(max_row_weights), int(max_prune_per_step), importance_eps,
                                           _p(self.out_deg, _i32p), _p(ptrs, _i32p), _p(cols, _i32p), _p(byts, _u8p),
                                           _p(tbr, _i32p), _p(tbc, _i32p), _p(tby, _u8p), C.byref(ntl),
                                           _p(rb, _u64p), _p(re_, _u64p), fail.ctypes.data_as(C.POINTER(C.c_int64)),
                                           None if b4 is None else C.byref(b4))
        n = int(ptrs[-1])
        k = int(ntl.value)
        self.load_csr(ptrs, cols[:n], bytes_=byts[:n])
        self.load_tiles(tbr[:k], tbc[:k], tby[:16 * k])
        if b4 is not None:
            R.ia, R.ea, R.ta = ([int(v) for v in a] for a in arrs)
            R.dropped = int(b4.dropped)
            self.b4_flags = fout[:max(1, k)].copy()
        if did == -4:
            raise MemoryError("std::bad_alloc")
        if did == -2:
            raise RuntimeError(synap_no_room_message(row, fail))
        if did == -3:
            raise RuntimeError(demote_no_room_message(fail))
        return bool(did), nxt

    def synap_step(self, importance_cutoff, max_row_weights, max_prune_per_step=8, importance_eps=1e-3,
                   reservations=None):
        cur = getattr(self, "synap_cursor", 0)
        did, self.synap_cursor = self.synap_row_step(cur, importance_cutoff, max_row_weights, max_prune_per_step,
                                                     importance_eps, reservations)
        return did

    def sampled_gradw(self, x, dy, threads=8, absmode=False):
        x = _c(np.atleast_2d(x), np.float32)
        dy = _c(np.atleast_2d(dy), np.float32)
        gs = np.zeros(max(1, int(self.row_elem_start[-1])), np.float32)
        gb = np.zeros(max(16, self.n_tiles * 16), np.float32)
        s = self._cstruct()
        lib().oracle_sampled_gradw(C.byref(s), _p(x, _f32p), _p(dy, _f32p), x.shape[0], _p(gs, _f32p),
                                   _p(gb, _f32p), threads, int(absmode))
        return gs[:int(self.row_elem_start[-1])], gb[:self.n_tiles * 16]

    def synapto_step(self, prune_frac, cand_r, cand_c, cand_v, cand_s=None, default_imp_code=1):
        cand_r, cand_c, cand_v = _c(cand_r, np.int32), _c(cand_c, np.int32), _c(cand_v, np.float32)
        cs = None if cand_s is None else _c(cand_s, np.float32)
        nnz = int(self.row_elem_start[-1])
        cap_s = nnz + len(cand_r) + 16 * self.n_tiles + 1
        cap_t = self.n_tiles + len(cand_r) + 1
        p = np.zeros(self.n_in + 1, np.int32)
        cols = np.zeros(cap_s, np.int32)
        byts = np.zeros(cap_s, np.uint8)
        tbr = np.zeros(cap_t, np.int32)
        tbc = np.zeros(cap_t, np.int32)
        tby = np.zeros(cap_t * 16, np.uint8)
        st = _SynStats()
        s = self._cstruct()
        rc = lib().oracle_synapto_step(C.byref(s), prune_frac, _p(cand_r, _i32p), _p(cand_c, _i32p),
                                       _p(cand_v, _f32p), _p(cs, _f32p), len(cand_r), default_imp_code,
                                       _p(p, _i32p), _p(cols, _i32p), _p(byts, _u8p), _p(tbr, _i32p),
                                       _p(tbc, _i32p), _p(tby, _u8p), C.byref(st))
        if rc != 0:
            raise RuntimeError("oracle synapto_step failed")
        ns, nt = st.n_scattered, st.n_tiles
        out = HostLayer(self.n_in, self.n_out, self.rank).set_scales(self.value_scale, self.output_scale)
        out.load_csr(p, cols[:ns], bytes_=byts[:ns])
        out.load_tiles(tbr[:nt], tbc[:nt], tby[:nt * 16])
        stats = {f[0]: getattr(st, f[0]) for f in _SynStats._fields_}
        return out, stats


class RefLayer:
    """The reference's own SparseLinearWeightsDelta, through ref_shim.cpp."""

    def __init__(self, n_in, n_out, ptrs, cols, w, imp=None, blank_fraction=0.2):
        self.n_in, self.n_out = int(n_in), int(n_out)
        R = reflib()
        self._keep = [_c(ptrs, np.int32), _c(cols, np.int32), _c(w, np.float32)]
        if imp is not None:
            self._keep.append(_c(imp, np.float32))
        self.h = R.ref_layer_new_blank(self.n_in, self.n_out, _p(self._keep[0], _i32p), _p(self._keep[1], _i32p),
                                       _p(self._keep[2], _f32p), _p(self._keep[3], _f32p) if imp is not None else None,
                                       float(blank_fraction))

    @classmethod
    def sll(cls, n_in, n_out, max_weights):
        """An empty layer as SparseLinearLayer(n_in, n_out, max_weights)
        constructs it (sili/cpu_backend.cpp:375-447): budgets and limits set."""
        self = cls.__new__(cls)
        self.n_in, self.n_out = int(n_in), int(n_out)
        self._keep = []
        self.h = reflib().ref_sll_new(self.n_in, self.n_out, int(max_weights))
        return self

    def _sll(self, rc):
        if rc != 0:
            raise MemoryError(reflib().ref_last_error().decode())
        return self

    def load_weights(self, ptrs, cols, w, imp=None):
        """SparseLinearLayer.load_weights (sili/cpu_backend.cpp:859-901)."""
        self._keep = [_c(ptrs, np.int32), _c(cols, np.int32), _c(w, np.float32)]
        imp = None if imp is None else _c(imp, np.float32)
        self._keep.append(imp)
        return self._sll(reflib().ref_sll_load_weights(self.h, _p(self._keep[0], _i32p), _p(self._keep[1], _i32p),
                                                       _p(self._keep[2], _f32p), _p(imp, _f32p)))

    def compact_layer(self):
        """SparseLinearLayer.compact (limits re-applied)."""
        return self._sll(reflib().ref_sll_compact(self.h))

    def expand_headroom(self, blank_fraction=0.2):
        return self._sll(reflib().ref_sll_expand(self.h, float(blank_fraction)))

    def expand_headroom_to(self, min_nnz_per_row, blank_fraction=0.2):
        return self._sll(reflib().ref_sll_expand_to(self.h, int(min_nnz_per_row), float(blank_fraction)))

    def equalize_to_capacity(self, target_elems_per_row, target_bytes_per_row=0):
        return self._sll(reflib().ref_sll_equalize_to_capacity(self.h, int(target_elems_per_row),
                                                               int(target_bytes_per_row)))

    def equalizer_step(self):
        return self._sll(reflib().ref_sll_equalizer_step(self.h))

    def layout(self):
        """The scattered DeltaCSRLayout: byte_start/elem_start [n_in+1],
        byte_end/elem_end [n_in]."""
        n = self.n_in
        bs, be = np.zeros(n + 1, np.uint64), np.zeros(max(n, 1), np.uint64)
        es, ee = np.zeros(n + 1, np.uint64), np.zeros(max(n, 1), np.uint64)
        reflib().ref_layer_layout(self.h, _p(bs, _u64p), _p(be, _u64p), _p(es, _u64p), _p(ee, _u64p))
        return dict(byte_start=bs, byte_end=be[:n], elem_start=es, elem_end=ee[:n])

    def block4_headroom(self, blank_fraction=0.2, min_slack_bytes=16):
        reflib().ref_layer_block4_headroom(self.h, float(blank_fraction), int(min_slack_bytes))
        return self

    def block4_reservations(self):
        """Per block row (ia, ea, ta, ui, ue, ut) as lists, and (dropped
        growth events, merge overflow events, overflow bytes, index budget,
        tile budget)."""
        R = reflib()
        n = R.ref_block4_reservations(self.h, *([None] * 7))
        arrs = [np.zeros(max(1, n), np.uint64) for _ in range(6)]
        out = np.zeros(5, np.uint64)
        R.ref_block4_reservations(self.h, *[_p(a, _u64p) for a in arrs], _p(out, _u64p))
        return tuple([int(v) for v in a[:n]] for a in arrs), tuple(int(v) for v in out)

    def block4_equalize_step(self):
        self._sll(reflib().ref_block4_equalize_step(self.h))

    def block4_expand(self, blank_fraction=0.2, min_slack_bytes=16):
        self._sll(reflib().ref_block4_expand(self.h, float(blank_fraction), int(min_slack_bytes)))

    def sll_load_dense_codes(self, wc, ic):
        wc, ic = _c(wc, np.uint8), _c(ic, np.uint8)
        self._sll(reflib().ref_sll_load_dense_codes(self.h, _p(wc, _u8p), _p(ic, _u8p)))

    def sll_put_tile(self, br, bc, tile16):
        t = _c(tile16, np.uint8)
        self._sll(reflib().ref_sll_put_tile(self.h, int(br), int(bc), _p(t, _u8p)))

    def build_probes(self, acc_in, acc_grad, k, per_row=False):
        acc_in, acc_grad = _c(acc_in, np.float32), _c(acc_grad, np.float32)
        reflib().ref_build_probes(self.h, _p(acc_in, _f32p), _p(acc_grad, _f32p), int(k), int(per_row))

    def get_probes(self):
        """(rows, cols, scores) of the probe count, and whether the probe index vectors are non-empty."""
        has = C.c_int(0)
        n = reflib().ref_get_probes(self.h, None, None, None, 0, C.byref(has))
        pr, pc, pv = np.zeros(max(n, 1), np.int32), np.zeros(max(n, 1), np.int32), np.zeros(max(n, 1), np.float32)
        reflib().ref_get_probes(self.h, _p(pr, _i32p), _p(pc, _i32p), _p(pv, _f32p), n, C.byref(has))
        return pr[:n], pc[:n], pv[:n], bool(has.value)

    def synap_row_step(self, current_row, importance_cutoff, max_row_weights, max_prune_per_step=8,
                       importance_eps=1e-3):
        row = C.c_int64(int(current_row))
        rc = reflib().ref_synap_row_step(self.h, C.byref(row), importance_cutoff, int(max_row_weights),
                                         int(max_prune_per_step), importance_eps)
        if rc == -2:
            msg = reflib().ref_last_error().decode()
            if msg == "std::bad_alloc":  # the budget (std::bad_alloc -> MemoryError in the binding)
                raise MemoryError(msg)
            raise RuntimeError(msg)
        return bool(rc), int(row.value)

    def out_degree(self):
        out = np.zeros(self.n_out, np.int32)
        reflib().ref_get_out_degree(self.h, _p(out, _i32p))
        return out

    def __del__(self):
        if getattr(self, "h", None):
            reflib().ref_layer_free(self.h)
            self.h = None

    def set_scales(self, vs, os_=None, rank=1):
        vs = _c(vs, np.float32)
        osv = None if os_ is None else _c(os_, np.float32)
        if reflib().ref_layer_set_scales(self.h, _p(vs, _f32p), _p(osv, _f32p), rank) != 0:
            raise ValueError("bad scale rank")
        return self

    def put_tile(self, br, bc, tile16):
        t = _c(tile16, np.uint8)
        reflib().ref_layer_put_tile(self.h, int(br), int(bc), _p(t, _u8p))

    def load_dense_codes(self, wc, ic):
        wc, ic = _c(wc, np.uint8), _c(ic, np.uint8)
        reflib().ref_layer_load_dense_codes(self.h, _p(wc, _u8p), _p(ic, _u8p))

    def compact(self):
        reflib().ref_layer_compact(self.h)

    def export(self):
        R = reflib()
        nb = R.ref_layer_export(self.h, None, None, None, None)
        n = R.ref_layer_nnz_scattered(self.h)
        bs = np.zeros(self.n_in + 1, np.uint64)
        es = np.zeros(self.n_in + 1, np.uint64)
        idx = np.zeros(max(1, nb), np.uint8)
        val = np.zeros(max(1, n), np.uint8)
        R.ref_layer_export(self.h, _p(bs, _u64p), _p(es, _u64p), _p(idx, _u8p), _p(val, _u8p))
        return bs, es, idx[:nb], val[:n]

    def export_tiles_packed(self):
        """(tile_is_sparse flags, stored tile bytes concatenated, per-block-row
        used bytes) as the reference's Block4Store holds them."""
        R = reflib()
        n = R.ref_layer_export_tiles_packed(self.h, None, None, None)
        nt = len(self.export_tiles()[0])
        flags = np.zeros(max(nt, 1), np.uint8)
        packed = np.zeros(max(n, 1), np.uint8)
        used = np.zeros((self.n_in + 3) // 4, np.uint64)
        R.ref_layer_export_tiles_packed(self.h, _p(flags, _u8p), _p(packed, _u8p), _p(used, _u64p))
        return flags[:nt], packed[:n], used

    def switch_point(self, set_to=-1):
        return int(reflib().ref_block4_switch_point(self.h, int(set_to)))

    def export_tiles(self):
        R = reflib()
        n = R.ref_layer_export_tiles(self.h, None, None, None)
        br = np.zeros(max(1, n), np.int32)
        bc = np.zeros(max(1, n), np.int32)
        t = np.zeros(max(16, 16 * n), np.uint8)
        R.ref_layer_export_tiles(self.h, _p(br, _i32p), _p(bc, _i32p), _p(t, _u8p))
        return br[:n], bc[:n], t[:16 * n]

    def combined(self):
        R = reflib()
        n = R.ref_layer_combined(self.h, None, None, None, None)
        p = np.zeros(self.n_in + 1, np.int32)
        ix = np.zeros(max(1, n), np.int32)
        w = np.zeros(max(1, n), np.float32)
        imp = np.zeros(max(1, n), np.float32)
        R.ref_layer_combined(self.h, _p(p, _i32p), _p(ix, _i32p), _p(w, _f32p), _p(imp, _f32p))
        return p, ix[:n], w[:n], imp[:n]

    def forward_dense(self, x, threads=1):
        x = _c(np.atleast_2d(x), np.float32)
        y = np.zeros((x.shape[0], self.n_out), np.float32)
        reflib().ref_forward_dense(self.h, _p(x, _f32p), x.shape[0], _p(y, _f32p), threads)
        return y

    def backward_dense(self, x, dy, threads=1):
        x = _c(np.atleast_2d(x), np.float32)
        dy = _c(np.atleast_2d(dy), np.float32)
        dx = np.zeros_like(x)
        ai = np.zeros(self.n_in, np.float32)
        ag = np.zeros(self.n_out, np.float32)
        reflib().ref_backward_dense(self.h, _p(x, _f32p), _p(dy, _f32p), x.shape[0], _p(dx, _f32p),
                                    _p(ai, _f32p), _p(ag, _f32p), threads)
        return dx, ai, ag

    def set_importance_scales(self, is_=None, ois=None):
        self._is = None if is_ is None else _c(is_, np.float32)
        self._ois = None if ois is None else _c(ois, np.float32)
        reflib().ref_layer_set_importance_scales(self.h, _p(self._is, _f32p), _p(self._ois, _f32p))

    def set_train_state(self, vs_imp=None, vs_mom=None, vs_step=None, os_imp=None, os_step=None, os_trainable=-1):
        u32p = C.POINTER(C.c_uint32)
        a = [None if v is None else _c(v, t) for v, t in ((vs_imp, np.float32), (vs_mom, np.float32),
                                                            (vs_step, np.uint32), (os_imp, np.float32),
                                                            (os_step, np.uint32))]
        reflib().ref_layer_set_train_state(self.h, _p(a[0], _f32p), _p(a[1], _f32p), _p(a[2], u32p),
                                           _p(a[3], _f32p), _p(a[4], u32p), int(os_trainable))

    def get_train_state(self, rank=1):
        nr, nc = self.n_in * rank, self.n_out * rank
        out = dict(value_scale=np.zeros(nr, np.float32), vs_importance=np.zeros(nr, np.float32),
                   vs_momentum=np.zeros(nr, np.float32), vs_step=np.zeros(nr, np.uint32),
                   output_scale=np.zeros(nc, np.float32), os_importance=np.zeros(nc, np.float32),
                   os_step=np.zeros(nc, np.uint32))
        u32p = C.POINTER(C.c_uint32)
        reflib().ref_layer_get_train_state(self.h, _p(out["value_scale"], _f32p), _p(out["vs_importance"], _f32p),
                                           _p(out["vs_momentum"], _f32p), _p(out["vs_step"], u32p),
                                           _p(out["output_scale"], _f32p), _p(out["os_importance"], _f32p),
                                           _p(out["os_step"], u32p))
        return out

    def backward_train(self, x, dy, lr, lr_per_row_nnz=False, damp_by_importance=True, beta2=0.999, eps=1e-8,
                       threads=1, variant="plain"):
        x = _c(np.atleast_2d(x), np.float32)
        dy = _c(np.atleast_2d(dy), np.float32)
        dx = np.zeros_like(x)
        ai = np.zeros(self.n_in, np.float32)
        ag = np.zeros(self.n_out, np.float32)
        reflib().ref_backward_train(self.h, _p(x, _f32p), _p(dy, _f32p), x.shape[0], _p(dx, _f32p), _p(ai, _f32p),
                                    _p(ag, _f32p), lr, int(lr_per_row_nnz), int(damp_by_importance), beta2, eps,
                                    threads, TRAIN_VARIANTS[variant])
        return dx, ai, ag

    def backward_sparse_train(self, x, dptrs, didx, dvals, batch, lr, lr_per_row_nnz=False, damp_by_importance=True,
                              beta2=0.999, eps=1e-8, threads=1, draw_seed=None):
        """draw_seed: reseeds the calling thread's stochastic-rounding RNG
        first (fp4_seed_stochastic_rng), which the block4 tiles' update draws
        from (with threads=1 the reference's loop runs on this thread)."""
        if draw_seed is not None:
            reflib().ref_seed_stochastic(int(draw_seed) & (2**64 - 1))
        x = _c(np.atleast_2d(x), np.float32)
        dptrs, didx, dvals = _c(dptrs, np.int32), _c(didx, np.int32), _c(dvals, np.float32)
        dx = np.zeros_like(x)
        ai = np.zeros(self.n_in, np.float32)
        ag = np.zeros(self.n_out, np.float32)
        reflib().ref_backward_sparse_train(self.h, _p(x, _f32p), _p(dptrs, _i32p), _p(didx, _i32p), _p(dvals, _f32p),
                                           batch, _p(dx, _f32p), _p(ai, _f32p), _p(ag, _f32p), lr,
                                           int(lr_per_row_nnz), int(damp_by_importance), beta2, eps, threads)
        return dx, ai, ag

    def forward_sparse(self, ptrs, idx, vals, batch, threads=1):
        ptrs, idx, vals = _c(ptrs, np.int32), _c(idx, np.int32), _c(vals, np.float32)
        y = np.zeros((batch, self.n_out), np.float32)
        reflib().ref_forward_sparse(self.h, _p(ptrs, _i32p), _p(idx, _i32p), _p(vals, _f32p), batch,
                                    _p(y, _f32p), threads)
        return y

    def backward_sparse(self, x, dptrs, didx, dvals, batch, threads=1):
        x = _c(np.atleast_2d(x), np.float32)
        dptrs, didx, dvals = _c(dptrs, np.int32), _c(didx, np.int32), _c(dvals, np.float32)
        dx = np.zeros_like(x)
        ai = np.zeros(self.n_in, np.float32)
        ag = np.zeros(self.n_out, np.float32)
        reflib().ref_backward_sparse(self.h, _p(x, _f32p), _p(dptrs, _i32p), _p(didx, _i32p), _p(dvals, _f32p),
                                     batch, _p(dx, _f32p), _p(ai, _f32p), _p(ag, _f32p), threads)
        return dx, ai, ag
