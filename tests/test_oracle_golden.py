"""CPU: pin the oracle (oracle/sili_oracle.cpp) against the reference's own
outputs (tests/golden/golden.npz, written by tests/golden/make_golden.py from
the reference's compiled headers), against closed forms, and against the
reference unit tests' hand-computed values."""
import os

import numpy as np
import pytest

from oracle import HostLayer, lib
from sili__new_amd.codec import fp4_decode_np, fp4_encode_np
from tests.util import assert_close_terms

G = np.load(os.path.join(os.path.dirname(__file__), "golden", "golden.npz"))

FP4_TABLE = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, np.nan, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0]


def test_fp4_decode_table_bits():
    got = np.array([lib().oracle_fp4_decode(c) for c in range(16)], np.float32).view(np.uint32)
    assert np.array_equal(got, G["fp4_table_bits"])
    assert G["fp4_table_bits"][8] == 0x7FC00000  # code 8 is NaN, not -0
    assert np.array_equal(fp4_decode_np(np.arange(16)).view(np.uint32), G["fp4_table_bits"])


def test_fp4_encode_matches_reference():
    v = G["fp4_values"]
    got = np.array([lib().oracle_fp4_encode(float(x)) for x in v], np.uint8)
    assert np.array_equal(got, G["fp4_codes"])
    assert np.array_equal(fp4_encode_np(v), G["fp4_codes"])


def test_fp4_encode_nearest_or_tied_and_kats():
    # tests/unit/test_fp4_bitshift.cpp:50-74: nearest-or-tied, never code 8
    rng = np.random.default_rng(1)
    v = np.concatenate([np.linspace(-8, 8, 16001, dtype=np.float32), rng.uniform(-10, 10, 200000).astype(np.float32)])
    codes = fp4_encode_np(v)
    table = np.array(FP4_TABLE, np.float64)
    finite = np.delete(np.arange(16), 8)
    best = np.min(np.abs(v[:, None].astype(np.float64) - table[finite][None, :]), axis=1)
    got = np.abs(v.astype(np.float64) - table[codes])
    assert not np.any(codes == 8)
    assert np.all(np.abs(got - best) < 1e-6)
    kat = {0.25: 0.5, 0.75: 1.0, 1.25: 1.5, 1.75: 2.0, 2.5: 3.0, 3.5: 4.0, 5.0: 6.0, -0.1: 0.0, 100.0: 6.0}
    for x, want in kat.items():
        assert table[lib().oracle_fp4_encode(x)] == want
    assert lib().oracle_fp4_encode(float("nan")) == 0


def test_fp4_encode_random_bit_patterns_agree():
    """Two independent restatements (C oracle, numpy codec) over 2^20 random
    fp32 bit patterns, NaN/Inf/subnormal included."""
    rng = np.random.default_rng(2)
    bits = rng.integers(0, 2**32, size=1 << 20, dtype=np.uint64).astype(np.uint32)
    v = bits.view(np.float32)
    out = np.zeros(len(v), np.uint8)
    import ctypes as C
    lib().oracle_fp4_encode_array(v.ctypes.data_as(C.POINTER(C.c_float)), len(v), out.ctypes.data_as(C.POINTER(C.c_uint8)))
    assert np.array_equal(out, fp4_encode_np(v))


def test_fp4_encode_bit_patterns_match_reference_digest():
    """The reference encoder's codes over 2^22 seeded random fp32 bit patterns
    (make_golden.py keeps their SHA-256)."""
    import ctypes as C
    import hashlib
    from sili__new_amd.synth import Stream
    v = Stream(7, 9).u64(1 << 22).astype(np.uint32).view(np.float32)
    out = np.zeros(len(v), np.uint8)
    lib().oracle_fp4_encode_array(v.ctypes.data_as(C.POINTER(C.c_float)), len(v), out.ctypes.data_as(C.POINTER(C.c_uint8)))
    assert hashlib.sha256(out.tobytes()).hexdigest() == str(G["fp4_bits_sha256"])
    assert hashlib.sha256(fp4_encode_np(v).tobytes()).hexdigest() == str(G["fp4_bits_sha256"])


def test_uleb_kats():
    import ctypes as C
    buf = np.zeros(8, np.uint8)
    for v, hx in zip(G["uleb_values"], G["uleb_hex"]):
        n = lib().oracle_uleb_encode(int(v), buf.ctypes.data_as(C.POINTER(C.c_uint8)))
        assert bytes(buf[:n]).hex() == str(hx)
    # DWARF 7.6 examples
    assert [str(h) for h in G["uleb_hex"][:6]] == ["00", "01", "7f", "8001", "ff7f", "808001"]


@pytest.mark.parametrize("name", ["kat", "edges", "cA", "cB", "cC", "b4"])
def test_structure_bit_exact(name):
    n_in, n_out = (int(v) for v in G[f"{name}_n"])
    imp = G[f"{name}_imp"] if f"{name}_imp" in G.files else None
    H = HostLayer(n_in, n_out).load_csr(G[f"{name}_ptrs"], G[f"{name}_cols"], w=G[f"{name}_w"], imp=imp)
    assert np.array_equal(H.row_byte_start, G[f"{name}_byte_start"])
    assert np.array_equal(H.row_elem_start, G[f"{name}_elem_start"])
    assert np.array_equal(H.idx[:H.index_bytes], G[f"{name}_idx"])
    assert np.array_equal(H.val[:H.nnz], G[f"{name}_val"])
    assert np.array_equal(H.decode_cols(), G[f"{name}_cols"])


def _golden_layer(name):
    n_in, n_out = (int(v) for v in G[f"{name}_n"])
    rank = int(G[f"{name}_rank"][0]) if f"{name}_rank" in G.files else 1
    H = HostLayer(n_in, n_out, rank).load_csr(G[f"{name}_ptrs"], G[f"{name}_cols"], w=G[f"{name}_w"])
    if f"{name}_tile_br" in G.files:
        H.load_tiles(G[f"{name}_tile_br"], G[f"{name}_tile_bc"], G[f"{name}_tiles_in"])
    vs = G[f"{name}_vs"] if f"{name}_vs" in G.files else None
    os_ = G[f"{name}_os"] if f"{name}_os" in G.files else None
    H.set_scales(vs, os_)
    return H


@pytest.mark.parametrize("name", ["cA", "cB", "cC", "b4"])
def test_compute_matches_reference(name):
    H = _golden_layer(name)
    x, dy = G[f"{name}_x"], G[f"{name}_dy"]
    B = x.shape[0]
    assert_close_terms(H.forward_dense(x), G[f"{name}_y"], H.forward_dense(x, absmode=True), "forward")
    dx, ai, ag = H.backward_dense(x, dy)
    assert_close_terms(dx, G[f"{name}_dx"], H.backward_dense(x, dy, absmode=True)[0], "dx")
    assert_close_terms(ai, G[f"{name}_acc_in"], ai, "acc_in")
    assert_close_terms(ag, G[f"{name}_acc_grad"], ag, "acc_grad")
    sx = (G[f"{name}_sx_ptrs"], G[f"{name}_sx_idx"], G[f"{name}_sx_vals"], B)
    assert_close_terms(H.forward_sparse(*sx), G[f"{name}_ys"], H.forward_sparse(*sx, absmode=True), "sparse fwd")
    sg = (G[f"{name}_sg_ptrs"], G[f"{name}_sg_idx"], G[f"{name}_sg_vals"], B)
    dxs, ai2, ag2 = H.backward_sparse(x, *sg)
    assert_close_terms(dxs, G[f"{name}_dxs"], H.backward_sparse(x, *sg, absmode=True)[0], "sparse grad dx")
    assert_close_terms(ag2, G[f"{name}_acc_grad_s"], ag2, "acc_grad sparse")
    p, ix, w, imp = H.absolute()
    assert np.array_equal(p, G[f"{name}_abs_ptrs"]) and np.array_equal(ix, G[f"{name}_abs_idx"])
    # decoded values compare as bits (code 8 decodes to the same NaN pattern)
    assert np.array_equal(w.view(np.uint32), G[f"{name}_abs_w"].view(np.uint32))
    assert np.array_equal(imp.view(np.uint32), G[f"{name}_abs_imp"].view(np.uint32))


def test_block4_store_matches_reference():
    H = _golden_layer("b4")
    assert np.array_equal(H.tile_br, G["b4_tiles_br_out"]) and np.array_equal(H.tile_bc, G["b4_tiles_bc_out"])
    assert np.array_equal(H.tiles[:16 * H.n_tiles], G["b4_tiles_out"])


def dense_codes_to_tiles(wc, ic, n_in, n_out):
    """Host restatement of load_dense_codes' tiling (delta_csr_memory.hpp:884-911),
    the same construction the C ABI performs."""
    brows, bcols = (n_in + 3) // 4, (n_out + 3) // 4
    br, bc, t = [], [], np.zeros((brows * bcols, 16), np.uint8)
    for i in range(brows):
        for j in range(bcols):
            k = i * bcols + j
            br.append(i)
            bc.append(j)
            for li in range(4):
                for lj in range(4):
                    r, c = i * 4 + li, j * 4 + lj
                    if r < n_in and c < n_out:
                        t[k, lj * 4 + li] = (int(wc[r * n_out + c]) | (int(ic[r * n_out + c]) << 4)) & 0xFF
    return np.array(br, np.int32), np.array(bc, np.int32), t.ravel()


def test_load_dense_codes_tiling_matches_reference():
    n_in, n_out = (int(v) for v in G["ldc_n"])
    br, bc, t = dense_codes_to_tiles(G["ldc_wc"], G["ldc_ic"], n_in, n_out)
    assert np.array_equal(br, G["ldc_br"]) and np.array_equal(bc, G["ldc_bc"])
    assert np.array_equal(t, G["ldc_tiles"])


@pytest.mark.parametrize("name", ["cA", "cB", "cC", "b4"])
def test_closed_form(name):
    """Forward/backward/grad-W against the dense product W_dense = dec*S in
    float64 (the reference tests' own check, test_disldo_synaptogenesis.cpp:36-38)."""
    H = _golden_layer(name)
    W = H.dense().astype(np.float64)
    x, dy = G[f"{name}_x"].astype(np.float64), G[f"{name}_dy"].astype(np.float64)
    bound_y = np.abs(x) @ np.abs(W)
    assert_close_terms(H.forward_dense(G[f"{name}_x"]), x @ W, bound_y, "y = xW")
    bound_dx = np.abs(dy) @ np.abs(W).T
    assert_close_terms(H.backward_dense(G[f"{name}_x"], G[f"{name}_dy"])[0], dy @ W.T, bound_dx, "dx = dy W^T")
    gs, gb = H.sampled_gradw(G[f"{name}_x"], G[f"{name}_dy"])
    full = x.T @ dy
    cols = H.decode_cols()
    rows = np.repeat(np.arange(H.n_in), np.diff(H.row_elem_start.astype(np.int64)))
    bound = np.abs(x).T @ np.abs(dy)
    assert_close_terms(gs, full[rows, cols], bound[rows, cols], "grad-W scattered")
    if H.n_tiles:
        li, lj = np.arange(16) % 4, np.arange(16) // 4
        r = (H.tile_br[:, None] * 4 + li[None, :])
        c = (H.tile_bc[:, None] * 4 + lj[None, :])
        ok = (r < H.n_in) & (c < H.n_out)
        want = np.where(ok, full[np.minimum(r, H.n_in - 1), np.minimum(c, H.n_out - 1)], 0.0)
        bnd = np.where(ok, bound[np.minimum(r, H.n_in - 1), np.minimum(c, H.n_out - 1)], 0.0)
        assert_close_terms(gb.reshape(-1, 16), want, bnd, "grad-W block4")


def test_reference_unit_kats():
    """test_disldo_synaptogenesis.cpp:14-89 and test_disldo_block4_*.cpp values."""
    H = HostLayer(3, 4).load_csr([0, 2, 3, 4], [0, 2, 1, 3], w=[1.5, -2.0, 0.5, 3.0])
    np.testing.assert_allclose(H.forward_dense([1.0, 0.6, 2.0])[0], [1.5, 0.3, -2.0, 6.0], atol=1e-6)
    dx, ai, ag = H.backward_dense([[1.0, 0.6, 2.0]], [[0.3, -0.5, 0.2, 0.4]])
    np.testing.assert_allclose(dx[0], [0.05, -0.25, 1.2], atol=1e-6)
    np.testing.assert_allclose(ai, [1.0, 0.6, 2.0], atol=1e-7)
    assert abs(ag[0] - 0.3) < 1e-7
    H = HostLayer(8, 8).load_csr([0, 1, 2, 2, 2, 2, 2, 2, 2], [5, 2], w=[2.0, -1.5])
    tile = np.zeros(16, np.uint8)
    tile[1 * 4 + 0] = 2 | (1 << 4)
    tile[3 * 4 + 2] = 1 | (1 << 4)
    H.load_tiles([0], [0], tile)
    x = np.zeros(8, np.float32)
    x[:3] = [3.0, 1.0, 2.0]
    want = np.zeros(8)
    want[[5, 2, 1, 3]] = [6.0, -1.5, 3.0, 1.0]
    np.testing.assert_allclose(H.forward_dense(x)[0], want, atol=1e-6)
    dy = np.zeros((1, 8), np.float32)
    dy[0, [5, 2, 1, 3]] = [0.7, -0.3, 0.4, -0.2]
    np.testing.assert_allclose(H.backward_dense(x, dy)[0][0, :3], [1.8, 0.45, -0.1], atol=1e-6)
