"""CPU: host-side logic -- seeded workload generators, the numpy FP4 codec,
the bench's algorithmic-bytes table and its one-GPU contract."""
import os
import subprocess
import sys

import numpy as np
import pytest

from oracle import lib as olib
from sili__new_amd.codec import fp4_decode_np, fp4_encode_np
from sili__new_amd.synth import Stream, make_config, poisson_lengths

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_stream_is_deterministic_and_distinct():
    a, b = Stream(5, 1).u64(1000), Stream(5, 1).u64(1000)
    assert np.array_equal(a, b)
    assert not np.array_equal(a, Stream(5, 2).u64(1000))
    u = Stream(9, 3).uniform(200000)
    assert 0.0 <= u.min() and u.max() < 1.0 and abs(u.mean() - 0.5) < 0.01
    z = Stream(9, 4).normal(200000)
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1.0) < 0.01


def test_poisson_lengths_statistics():
    L = poisson_lengths(Stream(1, 1), 200000, 164.0)
    assert abs(L.mean() - 164.0) < 0.2 and abs(L.var() - 164.0) < 3.0


@pytest.mark.parametrize("idx", [0, 1, 2, 3])
def test_configs_small_are_wellformed(idx):
    wl = make_config(idx, scale=0.0625)
    assert wl.n_in > 0 and wl.n_out > 0
    if wl.cols is not None:
        assert wl.ptrs[0] == 0 and wl.ptrs[-1] == len(wl.cols)
        for r in range(wl.n_in):
            seg = wl.cols[wl.ptrs[r]:wl.ptrs[r + 1]]
            assert np.all(np.diff(seg) > 0) and (len(seg) == 0 or (seg[0] >= 0 and seg[-1] < wl.n_out))
        # per-row quantizer: max |q| per non-empty row is 6 (s_r = max|w| / 6)
        for r in np.flatnonzero(np.diff(wl.ptrs))[:50]:
            assert np.isclose(np.abs(wl.q[wl.ptrs[r]:wl.ptrs[r + 1]]).max(), 6.0, rtol=1e-6)
    if wl.tile_br is not None:
        key = wl.tile_br.astype(np.int64) * (wl.n_out // 4) + wl.tile_bc
        assert np.all(np.diff(key) > 0)
        assert np.all((wl.tile_bytes >> 4) == 1)
    b = make_config(idx, scale=0.0625)
    assert b.nnz == wl.nnz and np.array_equal(b.x, wl.x)


def test_bench_workload_is_pinned():
    # the bench line is quoted on this exact synthetic matrix
    wl = make_config(1)
    assert (wl.n_in, wl.n_out, wl.batch) == (8192, 8192, 64)
    assert wl.nnz == 1343538


def test_codec_matches_oracle_on_bit_patterns():
    rng = np.random.default_rng(3)
    bits = rng.integers(0, 2**32, 20000, dtype=np.uint64).astype(np.uint32)
    v = bits.view(np.float32)
    want = np.array([olib().oracle_fp4_encode(float(x)) for x in v], np.uint8)
    assert np.array_equal(fp4_encode_np(v), want)
    codes = np.arange(16, dtype=np.uint8)
    dec = fp4_decode_np(codes)
    want_dec = np.array([olib().oracle_fp4_decode(int(c)) for c in codes], np.float32)
    assert np.array_equal(dec.view(np.uint32), want_dec.view(np.uint32))


def test_algorithmic_bytes_table():
    sys.path.insert(0, ROOT)
    import bench
    info = {"nnz_scattered": 1000, "index_bytes": 1100}
    t = bench.algorithmic(info, 64, 32, 8)
    base = 1000 + 1100 + 8 * 65 + 4 * (64 + 32)
    assert t["fwd:gather"] == base + 4 * 8 * 64 + 4 * 8 * 32
    assert t["bwd:sddmm"] == 1100 + 8 * 65 + 4 * 8 * 64 + 4 * 8 * 32 + 4 * 1000
    assert t["fwd:transpose"] == 8 * 8 * 64
    assert t["bwd:gather_gradw"] == base + 4 * 8 * 32 + 2 * 4 * 8 * 64 + 4 * 1000


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stdout


def test_uleb_row_bytes_matches_oracle_encoding():
    sys.path.insert(0, ROOT)
    import bench
    from oracle import HostLayer
    # empty rows first, in the middle and last; deltas across every varint length
    ptrs = np.array([0, 0, 3, 3, 6, 6], np.int32)
    cols = np.array([0, 127, 128, 5, 16384, 2**21 + 7], np.int32)
    H = HostLayer(5, 2**22).load_csr(ptrs, cols, w=np.ones(6, np.float32))
    assert np.array_equal(bench.uleb_row_bytes(ptrs, cols), np.diff(H.row_byte_start.astype(np.int64)))
    wl = make_config(2, scale=0.03125)
    H = HostLayer(wl.n_in, wl.n_out).load_csr(wl.ptrs, wl.cols, w=wl.q)
    assert np.array_equal(bench.uleb_row_bytes(wl.ptrs, wl.cols), np.diff(H.row_byte_start.astype(np.int64)))
