// wave.hpp -- wave64 primitives for gfx950: prefix scans and the ULEB128
// chunk decoder shared by every kernel that walks a delta-CSR stream.
#pragma once

#include "common.hpp"

namespace sili {

__device__ __forceinline__ uint32_t lane_id() { return __lane_id(); }

__device__ __forceinline__ uint32_t uniform(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_readfirstlane((int)v);
}

// Make this wave's LDS writes visible to its own later LDS reads (other lanes).
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Inclusive prefix sum over the 64 lanes.
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t x) {
    const uint32_t lane = lane_id();
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const uint32_t t = __shfl_up(x, d, 64);
        if (lane >= (uint32_t)d) x += t;
    }
    return x;
}

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) x += __shfl_xor(x, d, 64);
    return x;
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
    const uint64_t below = lane ? (~0ull >> (64u - lane)) : 0ull;
    const uint64_t prevT = T & below;
    // first byte of this lane's varint: one past the previous terminator
    const uint32_t s = prevT ? (64u - (uint32_t)__clzll(prevT)) : 0u;
    const uint32_t len = lane - s + 1u;
    const uint32_t b1 = __shfl_up(b, 1, 64), b2 = __shfl_up(b, 2, 64);
    const uint32_t b3 = __shfl_up(b, 3, 64), b4 = __shfl_up(b, 4, 64);
    // little-endian 7-bit groups: the terminator holds the most significant one
    uint32_t v = b & 0x7Fu;
    v = len > 1u ? ((v << 7) | (b1 & 0x7Fu)) : v;
    v = len > 2u ? ((v << 7) | (b2 & 0x7Fu)) : v;
    v = len > 3u ? ((v << 7) | (b3 & 0x7Fu)) : v;
    v = len > 4u ? ((v << 7) | (b4 & 0x7Fu)) : v;
    v = term ? v : 0u;
    ch.col = carry + wave_incl_scan(v);
    ch.rank = (uint32_t)__popcll(prevT);
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
