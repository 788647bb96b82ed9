"""Write tests/golden/golden.npz from the REFERENCE's own compiled code.

Runs in the build container only: it needs oracle/_ref/libsili_ref.so, which
oracle/Makefile compiles in place from the reference's headers
(sili/lib/headers, through oracle/ref_shim.cpp).  The fixtures are data
(inputs and the reference's outputs), small enough to commit; the tests read
them with numpy.load (no pickle).

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import os
import sys

import hashlib

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import RefLayer, reflib  # noqa: E402
from sili__new_amd.synth import Stream  # noqa: E402


def rand_csr(st: Stream, n_in: int, n_out: int, density: float, empty_rows=()):
    mask = st.uniform(n_in * n_out).reshape(n_in, n_out) < density
    for r in empty_rows:
        mask[r] = False
    ptrs = np.concatenate([[0], np.cumsum(mask.sum(1))]).astype(np.int32)
    cols = np.nonzero(mask)[1].astype(np.int32)
    return ptrs, cols


def fp4_cases(out):
    R = reflib()
    st = Stream(7, 1)
    vals = np.concatenate([
        np.array([0.0, -0.0, 0.25, -0.25, 0.2499999, 0.75, -0.75, 0.7499999, 1.0, 1.25, -1.25, 1.75, -1.75,
                  2.5, -2.5, 3.5, -3.5, 5.0, -5.0, 6.0, 7.0, 100.0, -100.0, np.inf, -np.inf, np.nan, 1e-30,
                  -1e-30, 0.5, -0.5], np.float32),
        (st.uniform(4000) * 20 - 10).astype(np.float32),
        st.normal(2000, 2.0),
    ]).astype(np.float32)
    out["fp4_values"] = vals
    out["fp4_codes"] = np.array([R.ref_fp4_encode(float(v)) for v in vals], np.uint8)
    out["fp4_table_bits"] = np.array([R.ref_fp4_table(c) for c in range(16)], np.float32).view(np.uint32)
    kat = np.array([0, 1, 127, 128, 16383, 16384, 2097151, 2097152, 268435455, 268435456, 4294967295],
                   np.uint64)
    buf = np.zeros(8, np.uint8)
    enc = []
    for v in kat:
        n = R.ref_uleb_encode(int(v), buf.ctypes.data_as(__import__("ctypes").POINTER(__import__("ctypes").c_uint8)))
        enc.append(bytes(buf[:n]).hex())
    out["uleb_values"] = kat
    out["uleb_hex"] = np.array(enc)
    # the reference encoder over 2^22 seeded random fp32 bit patterns (NaN,
    # Inf, subnormals included), kept as a SHA-256 of the code bytes
    bits = Stream(7, 9).u64(1 << 22).astype(np.uint32)
    codes = np.array([R.ref_fp4_encode(float(v)) for v in bits.view(np.float32)], np.uint8)
    out["fp4_bits_sha256"] = np.array(hashlib.sha256(codes.tobytes()).hexdigest())


def structure_case(out, name, n_in, n_out, ptrs, cols, w, imp=None):
    R = RefLayer(n_in, n_out, ptrs, cols, w, imp)
    R.compact()
    bs, es, idx, val = R.export()
    out[f"{name}_n"] = np.array([n_in, n_out], np.int64)
    out[f"{name}_ptrs"], out[f"{name}_cols"], out[f"{name}_w"] = ptrs, cols, np.asarray(w, np.float32)
    if imp is not None:
        out[f"{name}_imp"] = np.asarray(imp, np.float32)
    out[f"{name}_byte_start"], out[f"{name}_elem_start"] = bs, es
    out[f"{name}_idx"], out[f"{name}_val"] = idx, val
    return R


def compute_case(out, name, R, st, n_in, n_out, B, vs, os_, rank, tiles=None):
    if vs is not None:
        R.set_scales(vs, os_, rank)
        out[f"{name}_vs"] = np.asarray(vs, np.float32)
        if os_ is not None:
            out[f"{name}_os"] = np.asarray(os_, np.float32)
        out[f"{name}_rank"] = np.array([rank])
    x = st.normal(B * n_in).reshape(B, n_in)
    x[st.uniform(B * n_in).reshape(B, n_in) < 0.2] = 0.0   # exact zeros exercise the skip
    dy = st.normal(B * n_out).reshape(B, n_out)
    out[f"{name}_x"], out[f"{name}_dy"] = x, dy
    out[f"{name}_y"] = R.forward_dense(x)
    dx, ai, ag = R.backward_dense(x, dy)
    out[f"{name}_dx"], out[f"{name}_acc_in"], out[f"{name}_acc_grad"] = dx, ai, ag
    # sparse input: ~30% of each batch row, sorted indices
    xp, xi, xv = [0], [], []
    for b in range(B):
        keep = np.nonzero(st.uniform(n_in) < 0.3)[0]
        xi.extend(keep.tolist())
        xv.extend(x[b, keep].tolist())
        xp.append(len(xi))
    xp, xi, xv = np.array(xp, np.int32), np.array(xi, np.int32), np.array(xv, np.float32)
    out[f"{name}_sx_ptrs"], out[f"{name}_sx_idx"], out[f"{name}_sx_vals"] = xp, xi, xv
    out[f"{name}_ys"] = R.forward_sparse(xp, xi, xv, B)
    gp, gi, gv = [0], [], []
    for b in range(B):
        keep = np.nonzero(st.uniform(n_out) < 0.4)[0]
        gi.extend(keep.tolist())
        gv.extend(dy[b, keep].tolist())
        gp.append(len(gi))
    gp, gi, gv = np.array(gp, np.int32), np.array(gi, np.int32), np.array(gv, np.float32)
    out[f"{name}_sg_ptrs"], out[f"{name}_sg_idx"], out[f"{name}_sg_vals"] = gp, gi, gv
    dxs, ai2, ag2 = R.backward_sparse(x, gp, gi, gv, B)
    out[f"{name}_dxs"], out[f"{name}_acc_in_s"], out[f"{name}_acc_grad_s"] = dxs, ai2, ag2
    p, ix, w, imp = R.combined()
    out[f"{name}_abs_ptrs"], out[f"{name}_abs_idx"], out[f"{name}_abs_w"], out[f"{name}_abs_imp"] = p, ix, w, imp


def main():
    out = {}
    fp4_cases(out)
    st = Stream(20261201, 99)

    # reference unit-test KAT (tests/unit/test_disldo_synaptogenesis.cpp:14-89)
    structure_case(out, "kat", 3, 4, np.array([0, 2, 3, 4], np.int32), np.array([0, 2, 1, 3], np.int32),
                   np.array([1.5, -2.0, 0.5, 3.0], np.float32))

    # structure edge cases: empty first/middle/last rows, column 0, 1..5-byte deltas
    n_out = 300_000_000
    cols = [[0], [], [1, 127, 128, 16383, 16384 + 16383, 2097151 + 16384 + 16383],
            [268435455], [0, 268435456 + 31], [], [5, 6, 7, 299_999_999]]
    ptrs = np.concatenate([[0], np.cumsum([len(c) for c in cols])]).astype(np.int32)
    flat = np.array([c for row in cols for c in row], np.int32)
    w = st.normal(len(flat), 2.0)
    imp = np.abs(st.normal(len(flat), 1.0))
    structure_case(out, "edges", len(cols), n_out, ptrs, flat, w, imp)

    # compute cases (rank 1 with row scales, rank 1 with row+col scales, rank 2)
    for name, n_in, n_out, B, dens, rank in (("cA", 96, 80, 3, 0.12, 1), ("cB", 64, 130, 5, 0.2, 1),
                                             ("cC", 50, 70, 4, 0.15, 2)):
        ptrs, cols = rand_csr(st, n_in, n_out, dens, empty_rows=(0, n_in // 2, n_in - 1))
        w = st.normal(len(cols), 2.5)
        R = structure_case(out, name, n_in, n_out, ptrs, cols, w)
        vs = (np.abs(st.normal(n_in * rank, 0.3)) + 0.01).astype(np.float32)
        os_ = None if name == "cA" else (np.abs(st.normal(n_out * rank, 0.5)) + 0.05).astype(np.float32)
        compute_case(out, name, R, st, n_in, n_out, B, vs, os_, rank)

    # block4: scattered entries outside the tiles plus hand-placed tiles
    # (tests/unit/test_disldo_block4_forward.cpp:21-68 pattern), ragged edges
    n_in, n_out = 22, 18
    tiles = [(0, 0), (0, 3), (1, 1), (2, 4), (4, 0), (5, 2), (5, 4)]
    covered = np.zeros((n_in, n_out), bool)
    for br, bc in tiles:
        covered[br * 4:br * 4 + 4, bc * 4:bc * 4 + 4] = True
    mask = (st.uniform(n_in * n_out).reshape(n_in, n_out) < 0.25) & ~covered
    ptrs = np.concatenate([[0], np.cumsum(mask.sum(1))]).astype(np.int32)
    cols = np.nonzero(mask)[1].astype(np.int32)
    w = st.normal(len(cols), 2.0)
    R = structure_case(out, "b4", n_in, n_out, ptrs, cols, w)
    tb = np.zeros((len(tiles), 16), np.uint8)
    for t, (br, bc) in enumerate(tiles):
        codes = (st.integers(16, 16)).astype(np.uint8)
        codes[codes == 8] = 7                        # no NaN weights here
        imps = st.integers(16, 16).astype(np.uint8)
        live = st.uniform(16) < 0.7
        tb[t] = np.where(live, codes | (imps << 4), 0)
        R.put_tile(br, bc, tb[t])
    out["b4_tile_br"] = np.array([t[0] for t in tiles], np.int32)
    out["b4_tile_bc"] = np.array([t[1] for t in tiles], np.int32)
    out["b4_tiles_in"] = tb.ravel()
    ebr, ebc, et = R.export_tiles()
    out["b4_tiles_br_out"], out["b4_tiles_bc_out"], out["b4_tiles_out"] = ebr, ebc, et
    vs = (np.abs(st.normal(n_in, 0.3)) + 0.01).astype(np.float32)
    os_ = (np.abs(st.normal(n_out, 0.5)) + 0.05).astype(np.float32)
    compute_case(out, "b4", R, st, n_in, n_out, 3, vs, os_, 1)

    # load_dense_codes (delta_csr_memory.hpp:841-945): every block becomes a tile
    n_in, n_out = 9, 10
    wc = st.integers(n_in * n_out, 16).astype(np.uint8)
    ic = st.integers(n_in * n_out, 16).astype(np.uint8)
    wc[st.uniform(n_in * n_out) < 0.5] = 0
    ic[st.uniform(n_in * n_out) < 0.5] = 0
    R = RefLayer(n_in, n_out, np.zeros(n_in + 1, np.int32), np.zeros(0, np.int32), np.zeros(0, np.float32))
    R.load_dense_codes(wc, ic)
    out["ldc_n"] = np.array([n_in, n_out], np.int64)
    out["ldc_wc"], out["ldc_ic"] = wc, ic
    br, bc, t = R.export_tiles()
    out["ldc_br"], out["ldc_bc"], out["ldc_tiles"] = br, bc, t

    # structural rules used by synaptogenesis, on the reference's primitives:
    # (1) promote: a window with one scattered synapse receives an insert
    n_in, n_out = 8, 12
    ptrs = np.array([0, 2, 3, 3, 3, 4, 4, 5, 5], np.int32)
    cols = np.array([1, 9, 2, 6, 0], np.int32)
    w = np.array([1.5, -2.0, 3.0, -0.5, 6.0], np.float32)
    imp = np.array([0.5, 1.0, 0.0, 2.0, 4.0], np.float32)
    R = RefLayer(n_in, n_out, ptrs, cols, w, imp)
    # prune the smallest |w| synapse (4,6), regrow (2,3): window (0,0) then
    # holds (0,1),(1,2),(2,3) and is promoted
    reflib().ref_row_remove_col(R.h, 4, 6)
    reflib().ref_row_insert_col(R.h, 2, 3, 3.0, 0.5)
    reflib().ref_maybe_promote(R.h, 2, 3)
    out["promote_in"] = np.concatenate([ptrs, cols]).astype(np.int32)
    out["promote_w"], out["promote_imp"] = w, imp
    p, ix, ww, ii = R.combined()
    out["promote_abs_ptrs"], out["promote_abs_idx"], out["promote_abs_w"], out["promote_abs_imp"] = p, ix, ww, ii
    br, bc, t = R.export_tiles()
    out["promote_br"], out["promote_bc"], out["promote_tiles"] = br, bc, t
    # (2) demote: zero two of the three live slots -> live 1 -> demote to scattered
    reflib().ref_zero_tile_slot(R.h, 1, 2)
    z = reflib().ref_zero_tile_slot(R.h, 2, 3)
    out["demote_live_after_zero"] = np.array([z], np.int32)
    reflib().ref_demote_tile(R.h, 0, 0)
    p, ix, ww, ii = R.combined()
    out["demote_abs_ptrs"], out["demote_abs_idx"], out["demote_abs_w"], out["demote_abs_imp"] = p, ix, ww, ii
    br, bc, t = R.export_tiles()
    out["demote_ntiles"] = np.array([len(br)], np.int32)

    # (3) demote by magnitude: a tile whose two smallest-|w| slots are pruned
    # (the bulk synaptogenesis policy picks exactly these) demotes its last
    # live slot; the reference's primitives applied in the same order
    n_in, n_out = 8, 8
    ptrs = np.array([0, 1, 1, 2, 2, 3, 3, 3, 3], np.int32)
    cols = np.array([6, 7, 5], np.int32)
    w = np.array([6.0, -4.0, 3.0], np.float32)
    R = RefLayer(n_in, n_out, ptrs, cols, w)
    tile = np.zeros(16, np.uint8)
    tile[0 * 4 + 0] = 1 | (2 << 4)     # (0,0) w 0.5  imp 1.0
    tile[1 * 4 + 2] = 9 | (1 << 4)     # (2,1) w -0.5 imp 0.5
    tile[2 * 4 + 1] = 8 | (4 << 4)     # (1,2) w NaN (code 8), imp 2: requantizes to 0 on demote
    R.put_tile(0, 0, tile)
    reflib().ref_zero_tile_slot(R.h, 0, 0)
    reflib().ref_zero_tile_slot(R.h, 2, 1)
    reflib().ref_demote_tile(R.h, 0, 0)
    out["dm_in"] = np.concatenate([ptrs, cols]).astype(np.int32)
    out["dm_w"], out["dm_tile"] = w, tile
    p, ix, ww, ii = R.combined()
    out["dm_abs_ptrs"], out["dm_abs_idx"], out["dm_abs_w"], out["dm_abs_imp"] = p, ix, ww, ii
    bs, es, idx, val = R.export()
    out["dm_byte_start"], out["dm_elem_start"], out["dm_idx"], out["dm_val"] = bs, es, idx, val

    path = os.path.join(HERE, "golden.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path}: {len(out)} arrays, {os.path.getsize(path)} bytes")


if __name__ == "__main__":
    main()
