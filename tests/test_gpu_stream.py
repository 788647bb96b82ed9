"""GPU: the batch-1 stream gather (a padded copy of the store cut into
1024-byte windows) against the CPU oracle.

The stream copy puts every row on a 16-byte boundary (zero-delta padding
entries in front, columns shifted by one so that column 0 reads a zero
input) and lays the value bytes out parallel to the index bytes; the kernel
places rows on lanes and combines per-row pieces with a segmented wave scan.
The layers here are built to hit what that design has to get right: rows of
every length from 1 entry up, empty rows (many of them in one window), rows
spanning many windows, multi-byte deltas (general decode) including a first
delta whose encoding grows with the column shift (127 -> 128), a partial
last window and an exactly full one, row scales on both sides, and
non-finite inputs.  Layers with non-finite weights keep the segment kernels.
The launcher's kernel choice is read back from the per-kernel profiler, so
each variant is known to have run."""
import ctypes as C

import numpy as np
import pytest

from oracle import HostLayer
from sili__new_amd.synth import per_row_quantize
from tests.util import assert_close_terms


def uleb_len(v):
    n = 1
    while v >= 128:
        v >>= 7
        n += 1
    return n


def row_bytes(cols):
    prev, n = 0, 0
    for c in cols:
        n += uleb_len(c - prev)
        prev = c
    return n


def mixed_rows(n_out, seed, total_mod=None):
    """Rows of 0 and 1..2900 entries, random columns (mixed delta lengths),
    rows whose first column is 127 (its shifted encoding needs 2 bytes), plus
    a final run of consecutive columns sized so that the stream length mod
    1024 is `total_mod` when given (the unpadded store's length)."""
    rng = np.random.default_rng(seed)
    lens = [0, 1, 2, 3, 5, 7, 8, 15, 16, 17, 0, 0, 31, 33, 64, 65, 127, 128, 129, 300, 0,
            505, 506, 507, 508, 509, 510, 511, 512, 513, 514, 700, 1020, 1021, 1022, 1023, 1024,
            1025, 1026, 1027, 1500, 2047, 2048, 2049, 2900]
    lens += list(rng.integers(1, 1200, size=60))
    rng.shuffle(lens)
    rows = [np.sort(rng.choice(n_out, size=min(int(n), n_out), replace=False)) for n in lens]
    rows += [np.arange(127, 127 + k) for k in (1, 3, 20)]
    if total_mod is not None:
        tot = sum(row_bytes(r) for r in rows)
        k = 16
        while (tot + k) % 1024 != total_mod:
            k += 1
        rows.append(np.arange(k))  # k one-byte deltas
    return rows


def transpose_rows(rows, n_out):
    pairs = [(c, r) for r, cs in enumerate(rows) for c in cs]
    out = [[] for _ in range(n_out)]
    for c, r in sorted(pairs):
        out[c].append(r)
    return [np.array(o, np.int64) for o in out]


def make_pair(hip, rows, n_out, seed=5, out_scales=True):
    n_in = len(rows)
    ptrs = np.concatenate([[0], np.cumsum([len(r) for r in rows])]).astype(np.int32)
    cols = (np.concatenate(rows) if ptrs[-1] else np.zeros(0)).astype(np.int32)
    rng = np.random.default_rng(seed)
    w = rng.normal(size=len(cols)).astype(np.float32)
    q, s = per_row_quantize(ptrs, w, n_in)
    os_ = rng.uniform(0.5, 2.0, size=n_out).astype(np.float32) if out_scales else None
    H = HostLayer(n_in, n_out)
    H.load_csr(ptrs, cols, w=q)
    H.set_scales(s, os_)
    L = hip.SparseLinearLayer(n_in, n_out, max(1, len(cols)))
    L.load_weights(ptrs, cols, q)
    L.set_value_scales(s)
    if os_ is not None:
        L.set_output_scales(os_)
    return H, L


@pytest.fixture(autouse=True)
def stream_always(monkeypatch):
    """Use the stream kernels on every store that allows them (by default
    only stores of >= 1 MiB of index bytes take them)."""
    monkeypatch.setenv("SILI_B1_STREAM", "2")
    yield


class Entry(C.Structure):
    _fields_ = [("name", C.c_char * 56), ("count", C.c_int64), ("total_ms", C.c_double),
                ("min_ms", C.c_double), ("max_ms", C.c_double)]


def kernels_run(hip, L, fn):
    """Run fn() with L's profiler on; return the profiled kernel names."""
    lib = C.CDLL(hip.LIB_PATH)
    lib.sili_profile_enable.argtypes = [C.c_void_p, C.c_int]
    lib.sili_profile_read.argtypes = [C.c_void_p, C.POINTER(Entry), C.c_int, C.POINTER(C.c_int)]
    h = C.c_void_p(L.handle)
    assert lib.sili_profile_enable(h, 1) == 0
    fn()
    buf = (Entry * 64)()
    n = C.c_int()
    assert lib.sili_profile_read(h, buf, 64, C.byref(n)) == 0
    assert lib.sili_profile_enable(h, 0) == 0
    return {buf[i].name.decode() for i in range(n.value)}


def check_fwd(H, L, x, what):
    y = L.forward_dense(x)
    assert_close_terms(y, H.forward_dense(x), H.forward_dense(x, absmode=True), what)


def check_bwd(H, L, x, g, what):
    L.forward_dense(x)
    dx = L.backward_dense(g, 0.0)
    assert_close_terms(dx, H.backward_dense(x, g)[0], H.backward_dense(x, g, absmode=True)[0], what)


def test_mixed_rows_design():
    """CPU check of the designed layers: the requested stream lengths mod
    1024 are met and short, empty and 127-first rows are present."""
    for mod in (None, 0, 37):
        rows = mixed_rows(3000, 1, mod)
        nb = [row_bytes(r) for r in rows]
        assert min(nb) == 0 and any(0 < b < 16 for b in nb)
        assert any(len(r) and r[0] == 127 for r in rows)
        if mod is not None:
            assert sum(nb) % 1024 == mod


@pytest.mark.gpu
@pytest.mark.parametrize("mod", [None, 0, 1, 1023])
def test_stream_canonical_and_shadow(hip, mod):
    n_out = 3000
    rows = mixed_rows(n_out, 2 + (mod or 0), mod)
    # canonical orientation: dx = W^T g at batch 1 gathers the designed rows
    H, L = make_pair(hip, rows, n_out)
    T = transpose_rows(rows, n_out)
    HT, LT = make_pair(hip, T, len(rows))
    rng = np.random.default_rng(9)
    for B in (1, 2, 4, 8):
        x = rng.normal(size=(B, len(rows))).astype(np.float32)
        g = rng.normal(size=(B, n_out)).astype(np.float32)
        names = kernels_run(hip, L, lambda: check_bwd(H, L, x, g, f"dx mod{mod} B{B}"))
        assert any(n.startswith("bwd:stream") for n in names), names
        assert L.info()["stream_canonical"]
        check_fwd(H, L, x, f"fwd mod{mod} B{B}")
        # shadow orientation: the transposed layer's forward gathers them
        xt = rng.normal(size=(B, n_out)).astype(np.float32)
        names = kernels_run(hip, LT, lambda: check_fwd(HT, LT, xt, f"T fwd mod{mod} B{B}"))
        assert any(n.startswith("fwd:stream") for n in names), names
        assert LT.info()["stream_shadow"]
        # a second call must not see the first call's output
        check_fwd(HT, LT, xt * 0.5, f"T fwd again mod{mod} B{B}")


@pytest.mark.gpu
def test_stream_nonfinite_inputs(hip):
    rows = mixed_rows(2000, 7)
    T = transpose_rows(rows, 2000)
    H, L = make_pair(hip, T, len(rows))
    x = np.random.default_rng(1).normal(size=(1, 2000)).astype(np.float32)
    x[0, 5] = np.inf
    x[0, 17] = -np.inf
    x[0, 40] = np.nan
    x[0, 100:120] = 0.0
    check_fwd(H, L, x, "non-finite x")


@pytest.mark.gpu
def test_stream_short_and_empty_rows(hip):
    """Rows of 1-20 entries, with runs of empty rows longer than a window
    holds lanes, and single-entry rows at column 0 and at the last column."""
    rng = np.random.default_rng(4)
    rows = []
    for r in range(3000):
        k = r % 23
        if k >= 21 or (500 <= r < 700):
            rows.append(np.zeros(0, np.int64))
        else:
            rows.append(np.sort(rng.choice(900, size=k, replace=False)))
    rows[10] = np.array([0])
    rows[11] = np.array([899])
    H, L = make_pair(hip, rows, 900)
    x = rng.normal(size=(1, len(rows))).astype(np.float32)
    g = rng.normal(size=(1, 900)).astype(np.float32)
    names = kernels_run(hip, L, lambda: check_bwd(H, L, x, g, "short rows dx"))
    assert any(n.startswith("bwd:stream") for n in names), names


@pytest.mark.gpu
def test_stream_not_used_with_nonfinite_weights(hip):
    """An infinite row scale (non-finite weights) needs the reference's skip
    of zero inputs: the segment kernels run."""
    rows = mixed_rows(2000, 5)
    T = transpose_rows(rows, 2000)
    n_in = len(T)
    ptrs = np.concatenate([[0], np.cumsum([len(r) for r in T])]).astype(np.int32)
    cols = np.concatenate(T).astype(np.int32)
    w = np.random.default_rng(2).normal(size=len(cols)).astype(np.float32)
    q, s = per_row_quantize(ptrs, w, n_in)
    s[7] = np.inf
    H = HostLayer(n_in, len(rows)).load_csr(ptrs, cols, w=q).set_scales(s)
    L = hip.SparseLinearLayer(n_in, len(rows), len(cols))
    L.load_weights(ptrs, cols, q)
    L.set_value_scales(s)
    x = np.random.default_rng(3).normal(size=(1, n_in)).astype(np.float32)
    x[0, ::7] = 0.0
    names = kernels_run(hip, L, lambda: check_fwd(H, L, x, "inf scale fwd"))
    assert L.info()["has_nonfinite"]  # (scales reach the device with the call)
    assert not any("stream" in n for n in names), names


def kernel_counts(hip, L, fn):
    lib = C.CDLL(hip.LIB_PATH)
    lib.sili_profile_enable.argtypes = [C.c_void_p, C.c_int]
    lib.sili_profile_read.argtypes = [C.c_void_p, C.POINTER(Entry), C.c_int, C.POINTER(C.c_int)]
    h = C.c_void_p(L.handle)
    assert lib.sili_profile_enable(h, 1) == 0
    fn()
    buf = (Entry * 64)()
    n = C.c_int()
    assert lib.sili_profile_read(h, buf, 64, C.byref(n)) == 0
    assert lib.sili_profile_enable(h, 0) == 0
    return {buf[i].name.decode(): buf[i].count for i in range(n.value)}


@pytest.mark.gpu
@pytest.mark.parametrize("n_in,B,xlds,want", [
    (3000, 1, "0", {"fwd:stream": 1}),
    (3000, 1, "1", {"fwd:stream_lds": 1}),
    (3000, 2, "1", {"fwd:stream_lds": 1}),
    (3000, 8, "1", {"fwd:stream_lds": 1}),
    (6000, 8, "1", {"fwd:stream_lds": 2}),    # input too wide for LDS at 8 columns: 2 column blocks
    (6000, 8, "0", {"fwd:stream": 1}),
    (6000, 4, "0", {"fwd:stream": 1}),
    (12000, 4, "-1", {"fwd:stream_lds": 2}),  # automatic choice: 2 column blocks
    (36000, 2, "1", {"fwd:stream_lds": 2}),
    (36000, 2, "0", {"fwd:stream": 1}),
    (42000, 2, "1", {"fwd:stream_lds": 3}),
    (100000, 8, "-1", {"fwd:stream": 1}),     # more than 16 blocks: through the cache
])
def test_stream_variants(hip, monkeypatch, n_in, B, xlds, want):
    """Each launch variant (input in LDS or through the cache, whole rows or
    column blocks) against the oracle, the variant read back from the
    profiler."""
    monkeypatch.setenv("SILI_STREAM_XLDS", xlds)
    n_out = 20000 if n_in < 10000 else 800
    L = hip.SparseLinearLayer(n_in, n_out, 1)
    L.load_synthetic(4242 + n_in, 0.05, 0.02, 0.5)
    ex = L.export_scattered()
    H = HostLayer(n_in, n_out).load_encoded(ex["row_byte_start"], ex["row_elem_start"], ex["idx"], ex["val"])
    H.set_scales(np.asarray(L.get_value_scales(), np.float32))
    x = np.random.default_rng(n_in + B).normal(size=(B, n_in)).astype(np.float32)
    got = kernel_counts(hip, L, lambda: check_fwd(H, L, x, f"synthetic {n_in}x{n_out} B{B}"))
    got = {k: v for k, v in got.items() if k in ("fwd:stream", "fwd:stream_lds")}
    assert got == want, got


@pytest.mark.gpu
def test_stream_column_blocks_designed_rows(hip):
    """Column blocks over the designed rows (canonical orientation, 60000
    columns: 2 blocks at batch 1, 13 at batch 8): block boundaries fall
    inside rows, between multi-byte deltas and in rows with a single entry."""
    n_out = 60000
    rows = mixed_rows(n_out, 11)
    rows += [np.array([4990, 4991, 4992, 9983, 9984]), np.array([59999]), np.array([0, 59999])]
    H, L = make_pair(hip, rows, n_out)
    rng = np.random.default_rng(12)
    for B in (1, 2, 4, 8):
        x = rng.normal(size=(B, len(rows))).astype(np.float32)
        g = rng.normal(size=(B, n_out)).astype(np.float32)
        got = kernel_counts(hip, L, lambda: check_bwd(H, L, x, g, f"blocked dx B{B}"))
        assert got.get("bwd:stream_lds", 0) >= 2, got
