// wave.hpp -- wave64 primitives for gfx950: prefix scans and the ULEB128
// chunk decoder shared by every kernel that walks a delta-CSR stream.
#pragma once

#include "common.hpp"

namespace sili {

__device__ __forceinline__ uint32_t lane_id() { return __lane_id(); }

__device__ __forceinline__ uint32_t uniform(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_readfirstlane((int)v);
}

// Workgroups of a launch are dispatched round-robin over the 8 XCDs
// (workgroup n runs on XCD n % 8), each XCD with its own L2.  xcd_block maps
// the hardware workgroup id to a logical one so that every XCD takes one
// contiguous range of logical blocks (XCD x: [x*q + min(x, r), ...) for
// nblocks = 8q + r, q + (x < r) of them); a bijection on [0, nblocks).
// Blocks on neighbouring rows then write their shares of an output cache
// line from the same L2.
__device__ __forceinline__ uint32_t xcd_block(uint32_t n, uint32_t nblocks) {
    const uint32_t q = nblocks >> 3, r = nblocks & 7u;
    const uint32_t x = n & 7u, k = n >> 3;
    return x * q + (x < r ? x : r) + k;
}

// Make this wave's LDS writes visible to its own later LDS reads (other lanes).
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// DPP lane moves (gfx9 encodings).  Lanes whose source falls outside the
// row (or rows not selected by ROW_MASK) read 0.  Call with all lanes active.
// (bound_ctrl set: an out-of-row source reads 0, the same as the old value 0
// gives, and the compiler then needs no zeroed register per move.)
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t x) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, CTRL, ROW_MASK, 0xF, true);
}
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_f32(float x) {
    return __builtin_bit_cast(float, dpp_u32<CTRL, ROW_MASK>(__builtin_bit_cast(uint32_t, x)));
}
constexpr int DPP_ROW_SHR1 = 0x111, DPP_ROW_SHR2 = 0x112, DPP_ROW_SHR4 = 0x114, DPP_ROW_SHR8 = 0x118;
constexpr int DPP_ROW_ROR1 = 0x121, DPP_ROW_ROR2 = 0x122, DPP_ROW_ROR4 = 0x124, DPP_ROW_ROR8 = 0x128;
constexpr int DPP_ROW_BCAST15 = 0x142, DPP_ROW_BCAST31 = 0x143;

// Inclusive prefix sum over the 64 lanes: Hillis-Steele inside each 16-lane
// row (row_shr 1,2,4,8), then row_bcast15 / row_bcast31 carry across rows.
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t x) {
    x += dpp_u32<DPP_ROW_SHR1>(x);
    x += dpp_u32<DPP_ROW_SHR2>(x);
    x += dpp_u32<DPP_ROW_SHR4>(x);
    x += dpp_u32<DPP_ROW_SHR8>(x);
    x += dpp_u32<DPP_ROW_BCAST15, 0xA>(x);
    x += dpp_u32<DPP_ROW_BCAST31, 0xC>(x);
    return x;
}

// Segmented inclusive scans over the 64 lanes: f != 0 marks the first lane of
// a segment (lane 0 always begins one).  The wave_incl_scan ladder with the
// operator (a, fa) . (b, fb) = (fb ? b : a + b, fa | fb) (lanes outside a
// DPP row read the identity (0, 0)).
template <int CTRL, int RM>
__device__ __forceinline__ void seg_step(float &v, uint32_t &f) {
    const float t = dpp_f32<CTRL, RM>(v);
    const uint32_t tf = dpp_u32<CTRL, RM>(f);
    v = f ? v : v + t;
    f |= tf;
}
template <int CTRL, int RM>
__device__ __forceinline__ void seg_step(uint32_t &v, uint32_t &f) {
    const uint32_t t = dpp_u32<CTRL, RM>(v);
    const uint32_t tf = dpp_u32<CTRL, RM>(f);
    v = f ? v : v + t;
    f |= tf;
}
template <typename T>
__device__ __forceinline__ T wave_seg_scan(T v, uint32_t f) {
    seg_step<DPP_ROW_SHR1, 0xF>(v, f);
    seg_step<DPP_ROW_SHR2, 0xF>(v, f);
    seg_step<DPP_ROW_SHR4, 0xF>(v, f);
    seg_step<DPP_ROW_SHR8, 0xF>(v, f);
    seg_step<DPP_ROW_BCAST15, 0xA>(v, f);
    seg_step<DPP_ROW_BCAST31, 0xC>(v, f);
    return v;
}
// Inclusive running maximum over the lanes.
__device__ __forceinline__ uint32_t wave_max_scan(uint32_t x) {
    x = max(x, dpp_u32<DPP_ROW_SHR1>(x));
    x = max(x, dpp_u32<DPP_ROW_SHR2>(x));
    x = max(x, dpp_u32<DPP_ROW_SHR4>(x));
    x = max(x, dpp_u32<DPP_ROW_SHR8>(x));
    x = max(x, dpp_u32<DPP_ROW_BCAST15, 0xA>(x));
    x = max(x, dpp_u32<DPP_ROW_BCAST31, 0xC>(x));
    return x;
}
// Bitwise OR over all 64 lanes (wave-uniform result).
__device__ __forceinline__ uint32_t wave_or_all(uint32_t x) {
    x |= dpp_u32<DPP_ROW_SHR1>(x);
    x |= dpp_u32<DPP_ROW_SHR2>(x);
    x |= dpp_u32<DPP_ROW_SHR4>(x);
    x |= dpp_u32<DPP_ROW_SHR8>(x);
    x |= dpp_u32<DPP_ROW_BCAST15, 0xA>(x);
    x |= dpp_u32<DPP_ROW_BCAST31, 0xC>(x);
    return (uint32_t)__builtin_amdgcn_readlane((int)x, 63);
}
// Value of the previous lane (lane 0 reads 0): DPP wave_shr:1.
__device__ __forceinline__ uint32_t wave_prev_u32(uint32_t x) { return dpp_u32<0x138>(x); }
__device__ __forceinline__ float wave_prev_f32(float x) { return dpp_f32<0x138>(x); }

// Sum over each aligned group of BL lanes (BL a power of two <= 64); the
// group's total lands in its last lane (lane % BL == BL-1).  Inside a row the
// steps rotate (row_ror 1, 2, 4, 8): the last lane of a group adds the same
// lanes in the same order as with row_shr, and since every lane has a source
// each step is one v_add_f32 with DPP (row_shr:8 took a separate move).
template <int BL>
__device__ __forceinline__ float group_sum_last(float v) {
    if constexpr (BL >= 2) v += dpp_f32<DPP_ROW_ROR1>(v);
    if constexpr (BL >= 4) v += dpp_f32<DPP_ROW_ROR2>(v);
    if constexpr (BL >= 8) v += dpp_f32<DPP_ROW_ROR4>(v);
    if constexpr (BL >= 16) v += dpp_f32<DPP_ROW_ROR8>(v);
    if constexpr (BL >= 32) v += dpp_f32<DPP_ROW_BCAST15, 0xA>(v);
    if constexpr (BL >= 64) v += dpp_f32<DPP_ROW_BCAST31, 0xC>(v);
    return v;
}

// Sum over all 64 lanes, broadcast to every lane.
__device__ __forceinline__ float wave_sum(float x) {
    x = group_sum_last<64>(x);
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), 63));
}

// One 64-byte window of a ULEB128 delta stream.  The window starts at a
// varint boundary `pos` whose preceding column is `carry`; bytes at or past
// `end` count as continuation bytes so they never terminate a varint.
// Each lane holding the last byte of a varint (a "terminator") gets that
// entry's absolute column and its rank among the window's entries.
struct Chunk {
    uint64_t T;     // terminator mask (wave-uniform)
    uint32_t col;   // absolute column (terminator lanes)
    uint32_t rank;  // entry rank within the window (terminator lanes)
    uint32_t v;     // the entry's column delta (terminator lanes), else 0
    bool term;
};

__device__ __forceinline__ Chunk decode_chunk(const uint8_t *__restrict__ idx, uint32_t pos,
                                              uint32_t end, uint32_t carry) {
    Chunk ch;
    const uint32_t lane = lane_id();
    const uint32_t p = pos + lane;
    const uint32_t b = (p < end) ? (uint32_t)idx[p] : 0x80u;
    const bool term = (b & 0x80u) == 0u;
    const uint64_t T = __ballot(term);
    // continuation flags of the 4 bytes before this lane, bit 3 = lane-1; the
    // window starts at a varint boundary, so positions before it read as 0
    // (two shifts: a single (~T << 4) would drop the flags of lanes 60-63)
    const uint64_t NT = ~T;
    const uint64_t E = lane >= 4u ? (NT >> (lane - 4u)) : (NT << (4u - lane));
    const uint32_t q = (uint32_t)E & 0xFu;
    const uint32_t t = ~q & 0xFu;                             // first non-continuation from the top
    const uint32_t run = t ? (uint32_t)__builtin_clz(t) - 28u : 4u;  // preceding bytes of this varint
    // little-endian 7-bit groups: the terminator holds the most significant one
    const uint32_t b1 = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)b, 0x138, 0xF, 0xF, false);   // wave_shr:1
    const uint32_t b2 = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)b1, 0x138, 0xF, 0xF, false);
    const uint32_t b3 = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)b2, 0x138, 0xF, 0xF, false);
    const uint32_t b4 = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)b3, 0x138, 0xF, 0xF, false);
    uint32_t v = b & 0x7Fu;
    v = run >= 1u ? ((v << 7) | (b1 & 0x7Fu)) : v;
    v = run >= 2u ? ((v << 7) | (b2 & 0x7Fu)) : v;
    v = run >= 3u ? ((v << 7) | (b3 & 0x7Fu)) : v;
    v = run >= 4u ? ((v << 7) | (b4 & 0x7Fu)) : v;
    v = term ? v : 0u;
    ch.col = carry + wave_incl_scan(v);
    ch.v = v;
    ch.rank = __builtin_amdgcn_mbcnt_hi((uint32_t)(T >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)T, 0u));
    ch.term = term;
    ch.T = T;
    return ch;
}

// Advance a decoder past a window: returns the new carry (column of the
// window's last entry); updates pos / ebase.  T must be non-zero.
__device__ __forceinline__ uint32_t chunk_advance(const Chunk &ch, uint32_t &pos, uint32_t &ebase) {
    const uint32_t hi = 63u - (uint32_t)__clzll(ch.T);
    const uint32_t carry = uniform((uint32_t)__shfl((int)ch.col, (int)hi, 64));
    pos += hi + 1u;
    ebase += (uint32_t)__popcll(ch.T);
    return carry;
}

// LDS copy of one segment's index bytes and value bytes (one per wave).
struct alignas(16) SegStage {
    uint32_t idx[SEG_BYTES_MAX / 4 + 4];
    uint32_t val[SEG_BYTES_MAX / 4 + 4];
};

// Copy bytes [begin, end) of a device buffer into dst as aligned dwords
// (every load in flight at once); `off` = position of `begin` in dst.  The
// device buffers carry >= 4 bytes of padding, so the last dword is in bounds.
__device__ __forceinline__ void stage_words(uint32_t *dst, const uint8_t *src_bytes, uint32_t begin,
                                            uint32_t end, uint32_t &off) {
    const uint32_t b0 = begin & ~3u;
    off = begin - b0;
    uint32_t nw = (end - b0 + 3u) >> 2;
    nw = nw < SEG_BYTES_MAX / 4 + 4 ? nw : SEG_BYTES_MAX / 4 + 4;
    const uint32_t *src = reinterpret_cast<const uint32_t *>(src_bytes + b0);
    for (uint32_t i = lane_id(); i < nw; i += 64u) dst[i] = src[i];
}

// Stage a segment and return the LDS byte views; pos/end become relative.
struct StagedSeg {
    const uint8_t *idx;  // idx[0] = first index byte of the segment
    const uint8_t *val;  // val[e - elem_begin] = value byte of entry e
    uint32_t end;        // index bytes in the segment
};
__device__ __forceinline__ StagedSeg stage_segment(SegStage &S, const uint8_t *idx, const uint8_t *val,
                                                   const SegDesc &sd) {
    uint32_t ioff = 0, voff = 0;
    stage_words(S.idx, idx, sd.byte_begin, sd.byte_end, ioff);
    if (val) stage_words(S.val, val, sd.elem_begin, sd.elem_end, voff);
    wave_lds_sync();
    StagedSeg g;
    g.idx = reinterpret_cast<const uint8_t *>(S.idx) + ioff;
    g.val = reinterpret_cast<const uint8_t *>(S.val) + voff;
    const uint32_t n = sd.byte_end - sd.byte_begin;
    g.end = n < SEG_BYTES_MAX ? n : SEG_BYTES_MAX;
    return g;
}

// Buffer resource over [base, base + bytes) for raw buffer loads; reads at
// offsets >= bytes return 0 (hardware range check).  bytes < 2^31.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ float4 buffer_load_f4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
}
__device__ __forceinline__ float buffer_load_f1(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0));
}
// An offset no buffer used here reaches: loads from it return 0.
constexpr uint32_t OOB_OFFSET = 0x80000000u;

// S(row, ent) = sum_k row_scale[row,k] * ent_scale[ent,k]; NULL = all ones
// (rank 1 only).  Components k >= 1 accumulate with fma.
__device__ __forceinline__ float scale_at(const ScaleView &sc, uint32_t row, uint32_t ent) {
    if (sc.rank == 1) {
        const float r = sc.row ? sc.row[row] : 1.0f;
        return sc.ent ? r * sc.ent[ent] : r;
    }
    const int rk = sc.rank;
    float s = sc.row[(size_t)row * rk] * sc.ent[(size_t)ent * rk];
    for (int k = 1; k < rk; ++k)
        s = __builtin_fmaf(sc.row[(size_t)row * rk + k], sc.ent[(size_t)ent * rk + k], s);
    return s;
}

template <int SKIP>
__device__ __forceinline__ bool skip_x(float x) {
    if constexpr (SKIP == SKIP_ZERO) return x == 0.0f;
    else if constexpr (SKIP == SKIP_POSZERO) return __builtin_bit_cast(uint32_t, x) == 0u;
    else return false;
}

}  // namespace sili
