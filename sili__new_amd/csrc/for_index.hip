// for_index.hip -- the group frame-of-reference (FOR) index of the canonical
// scattered store (prototypes/for_delta_encoding/README.md:18-40): a derived
// device copy of the column indices in which every column decodes as
// group start + its fixed-width offset, with no dependency on the columns
// before it.  The ULEB128 stream stays the store's source of truth; this copy
// is built from it on request and dropped whenever the store is rebuilt.
#include "../../include/sili_hip.h"
#include "layer.hpp"
#include "wave.hpp"

#include <cstring>  // host memset, needed before rocprim's headers

#include <rocprim/rocprim.hpp>

namespace sili {

namespace {

constexpr unsigned TPB = 256;
inline unsigned nblk(int64_t n) { return (unsigned)((n + TPB - 1) / TPB); }

__device__ __forceinline__ uint32_t tier_of(uint32_t maxoff) { return maxoff < 256u ? 0u : (maxoff < 65536u ? 1u : 2u); }
__device__ __forceinline__ uint32_t width_of(uint32_t tier) { return tier == 0u ? 1u : (tier == 1u ? 2u : 4u); }

// groups per row
__global__ void k_for_row_groups(const uint32_t *__restrict__ elem_start, int64_t rows, uint32_t G,
                                 uint32_t *__restrict__ cnt) {
    const int64_t r = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (r > rows) return;
    cnt[r] = r < rows ? (elem_start[r + 1] - elem_start[r] + G - 1u) / G : 0u;
}

// Per group: its row (largest r with row_group[r] <= g), first entry, start
// column, and byte length 1 + G * width.
__global__ void k_for_group_meta(const uint32_t *__restrict__ row_group, int64_t rows,
                                 const uint32_t *__restrict__ elem_start, const int32_t *__restrict__ cols,
                                 int64_t ngroups, uint32_t G, uint32_t *__restrict__ group_base,
                                 uint32_t *__restrict__ group_elem, uint32_t *__restrict__ len) {
    const int64_t g = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (g >= ngroups) return;
    int64_t lo = 0, hi = rows - 1;
    while (lo < hi) {
        const int64_t mid = (lo + hi + 1) >> 1;
        if ((int64_t)row_group[mid] <= g) lo = mid;
        else hi = mid - 1;
    }
    const int64_t r = lo;
    const uint32_t j = (uint32_t)(g - row_group[r]);
    const uint32_t e0 = elem_start[r] + j * G, re = elem_start[r + 1];
    const uint32_t e1 = e0 + G < re ? e0 + G : re;
    const uint32_t base = j == 0u ? 0u : (uint32_t)cols[e0 - 1u];
    group_base[g] = base;
    group_elem[g] = e0;
    len[g] = 1u + G * width_of(tier_of((uint32_t)cols[e1 - 1u] - base));
}

// One thread per (group, slot): slot 0 also writes the tier byte.
__global__ void k_for_group_write(const uint32_t *__restrict__ group_pos, const uint32_t *__restrict__ group_base,
                                  const uint32_t *__restrict__ group_elem, const int32_t *__restrict__ cols,
                                  int64_t ngroups, uint32_t G, uint8_t *__restrict__ out) {
    const int64_t t = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (t >= ngroups * (int64_t)G) return;
    const int64_t g = t / G;
    const uint32_t k = (uint32_t)(t % G);
    const uint32_t e0 = group_elem[g], n = group_elem[g + 1] - e0;
    const uint32_t base = group_base[g];
    const uint32_t maxoff = (uint32_t)cols[e0 + n - 1u] - base;
    const uint32_t tier = tier_of(maxoff), w = width_of(tier);
    const uint32_t off = k < n ? (uint32_t)cols[e0 + k] - base : maxoff;
    uint8_t *p = out + group_pos[g];
    if (k == 0u) p[0] = (uint8_t)tier;
    p += 1u + k * w;
    for (uint32_t b = 0; b < w; ++b) p[b] = (uint8_t)(off >> (8u * b));
}

__global__ void k_set_u32(uint32_t *__restrict__ p, uint32_t v) { *p = v; }

// Decode: one thread per (group, slot), 32-bit index math (G a power of
// two); column = group start + offset.  The group's tier byte and its three
// index words are shared by its G threads (cache hits after the first).
template <uint32_t G>
__global__ __launch_bounds__(TPB) void k_for_decode(const uint8_t *__restrict__ bytes,
                                                    const uint32_t *__restrict__ group_pos,
                                                    const uint32_t *__restrict__ group_base,
                                                    const uint32_t *__restrict__ group_elem, uint32_t nslots,
                                                    int32_t *__restrict__ cols) {
    const uint32_t t = blockIdx.x * TPB + threadIdx.x;
    if (t >= nslots) return;
    const uint32_t g = t / G, k = t % G;
    const uint32_t e0 = group_elem[g];
    if (k >= group_elem[g + 1] - e0) return;
    const uint8_t *p = bytes + group_pos[g];
    const uint32_t tier = p[0];
    uint32_t off;
    if (tier == 0u) {
        off = p[1u + k];
    } else if (tier == 1u) {
        off = (uint32_t)p[1u + 2u * k] | ((uint32_t)p[2u + 2u * k] << 8);
    } else {
        const uint8_t *q = p + 1u + 4u * k;
        off = (uint32_t)q[0] | ((uint32_t)q[1] << 8) | ((uint32_t)q[2] << 16) | ((uint32_t)q[3] << 24);
    }
    cols[e0 + k] = (int32_t)(group_base[g] + off);
}

// Decode, one thread per group (G = 8 or 16): the group's bytes
// [pos, pos + 1 + G*w) are read as aligned dwords, all in flight at once, and
// realigned with v_alignbyte; every offset is then a fixed byte slice.  The
// byte buffer carries >= 4 bytes of padding past its last group, so the last
// aligned dword stays in bounds.
template <uint32_t G>
__global__ __launch_bounds__(TPB) void k_for_decode_tg(const uint8_t *__restrict__ bytes,
                                                       const uint32_t *__restrict__ group_pos,
                                                       const uint32_t *__restrict__ group_base,
                                                       const uint32_t *__restrict__ group_elem, uint32_t ngroups,
                                                       int32_t *__restrict__ cols) {
    constexpr uint32_t ND = (3u + 1u + 4u * G + 3u) / 4u + 1u;  // aligned dwords covering the widest group
    const uint32_t g = blockIdx.x * TPB + threadIdx.x;
    if (g >= ngroups) return;
    const uint32_t pos = group_pos[g], base = group_base[g];
    const uint32_t e0 = group_elem[g], n = group_elem[g + 1] - e0;
    const uint32_t a = pos & 3u;
    const uint32_t *src = reinterpret_cast<const uint32_t *>(bytes + (pos - a));
    // the tier (the group's first byte) sets how many dwords the group spans
    const uint32_t w0 = src[0];
    const uint32_t tier = (w0 >> (8u * a)) & 0xFFu;
    const uint32_t w = tier == 0u ? 1u : (tier == 1u ? 2u : 4u);
    const uint32_t nd = (a + 1u + G * w + 3u) / 4u;
    uint32_t dw[ND + 1];
    dw[0] = w0;
#pragma unroll
    for (uint32_t j = 1; j < ND + 1; ++j) dw[j] = j < nd ? src[j] : 0u;
    // gb[j] = group bytes [4j, 4j + 4)
    uint32_t gb[ND];
#pragma unroll
    for (uint32_t j = 0; j < ND; ++j) gb[j] = __builtin_amdgcn_alignbyte(dw[j + 1], dw[j], a);
    int32_t *out = cols + e0;
#pragma unroll
    for (uint32_t k = 0; k < G; ++k) {
        uint32_t off;
        if (tier == 0u) {  // offset k at byte 1 + k
            off = (gb[(1u + k) / 4u] >> (8u * ((1u + k) % 4u))) & 0xFFu;
        } else if (tier == 1u) {
            const uint32_t lo = (gb[(1u + 2u * k) / 4u] >> (8u * ((1u + 2u * k) % 4u))) & 0xFFu;
            const uint32_t hi = (gb[(2u + 2u * k) / 4u] >> (8u * ((2u + 2u * k) % 4u))) & 0xFFu;
            off = lo | (hi << 8);
        } else {
            off = __builtin_amdgcn_alignbyte(gb[(1u + 4u * k) / 4u + 1u], gb[(1u + 4u * k) / 4u], 1u);
        }
        if (k < n) out[k] = (int32_t)(base + off);
    }
}

// Decode, one wave per 64 / G groups and one lane per slot.  The wave's
// groups are contiguous in the byte stream: at most 64/G * (1 + 4G) bytes
// (267 with the alignment), so lane l loads the aligned dwords D0 + l and
// D0 + 64 + l once, coalesced (indices clamped to the buffer; the clamped
// words are never selected for a byte in use).  Each lane then takes the two
// dwords that hold its offset from the lanes that loaded them (__shfl), and
// realigns them to its byte.  The group's tier byte and its three index words
// are per-lane loads that the wave's lanes share (4 addresses per wave at G =
// 16).  G from 8 to 64.
template <uint32_t G>
__global__ __launch_bounds__(TPB) void k_for_decode_wave(const uint8_t *__restrict__ bytes, uint32_t ndw,
                                                         const uint32_t *__restrict__ group_pos,
                                                         const uint32_t *__restrict__ group_base,
                                                         const uint32_t *__restrict__ group_elem, uint32_t ngroups,
                                                         int32_t *__restrict__ cols) {
    constexpr uint32_t GPW = 64u / G;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t g0 = ((blockIdx.x * TPB + threadIdx.x) >> 6) * GPW;
    if (g0 >= ngroups) return;  // the whole wave
    const uint32_t g = g0 + lane / G, k = lane % G;
    const bool gv = g < ngroups;
    const uint32_t gg = gv ? g : g0;
    const uint32_t pos = group_pos[gg], base = group_base[gg], e0 = group_elem[gg];
    const uint32_t n = group_elem[gg + 1] - e0;
    const uint32_t pos0 = (uint32_t)__builtin_amdgcn_readfirstlane((int)pos);  // lane 0: group g0
    const uint32_t D0 = pos0 >> 2;
    const uint32_t *dw = reinterpret_cast<const uint32_t *>(bytes);
    const uint32_t wa = dw[min(D0 + lane, ndw - 1u)], wb = dw[min(D0 + 64u + lane, ndw - 1u)];
    const uint32_t tier = bytes[pos];
    const uint32_t w = tier == 0u ? 1u : (tier == 1u ? 2u : 4u);
    const uint32_t rb = pos - 4u * D0 + 1u + k * w;  // this slot's first byte, from the window's start
    const uint32_t di = rb >> 2;                     // < 67
    const uint32_t la = (uint32_t)__shfl((int)wa, (int)(di & 63u), 64), lb = (uint32_t)__shfl((int)wb, (int)(di & 63u), 64);
    const uint32_t ha = (uint32_t)__shfl((int)wa, (int)((di + 1u) & 63u), 64),
                   hb = (uint32_t)__shfl((int)wb, (int)((di + 1u) & 63u), 64);
    const uint32_t lo = di < 64u ? la : lb, hi = di + 1u < 64u ? ha : hb;
    const uint32_t v = __builtin_amdgcn_alignbyte(hi, lo, rb & 3u);
    const uint32_t off = w == 4u ? v : (v & ((1u << (8u * w)) - 1u));
    if (gv && k < n) cols[e0 + k] = (int32_t)(base + off);
}

void scan_u32(const uint32_t *in, uint32_t *out, int64_t n, DevBuf<uint8_t> &temp, hipStream_t st) {
    size_t bytes = 0;
    SILI_HIP(rocprim::exclusive_scan(nullptr, bytes, in, out, uint32_t(0), (size_t)n, rocprim::plus<uint32_t>(), st));
    if (bytes + 16 > temp.n) temp.ensure(bytes + 16);
    SILI_HIP(rocprim::exclusive_scan(temp.p, bytes, in, out, uint32_t(0), (size_t)n, rocprim::plus<uint32_t>(), st));
}

}  // namespace

void build_for_index(Layer &L, int G) {
    if (G != 8 && G != 16 && G != 32 && G != 64)
        throw_error(SILI_ERR_INVALID, "build_for_index: group size must be 8, 16, 32 or 64");
    DScatter &W = L.W;
    DFor &F = W.fidx;
    hipStream_t st = L.stream;
    ProfScope ps("for_build", st);
    const int64_t rows = W.rows, N = W.nnz;
    DevBuf<int32_t> cols;
    DevBuf<uint32_t> cnt, len;
    DevBuf<uint8_t> temp;
    cols.ensure((size_t)N + 1);
    if (N > 0) launch_decode(W.plan(), ScaleView{nullptr, nullptr, 1}, cols.p, nullptr, nullptr, st);
    cnt.ensure((size_t)rows + 1);
    F.row_group.ensure((size_t)rows + 1);
    launch(k_for_row_groups, dim3(nblk(rows + 1)), dim3(TPB), 0, st, (const uint32_t *)W.elem_start.p, rows,
           (uint32_t)G, cnt.p);
    scan_u32(cnt.p, F.row_group.p, rows + 1, temp, st);
    uint32_t ng = 0;
    SILI_HIP(hipMemcpyAsync(&ng, F.row_group.p + rows, 4, hipMemcpyDeviceToHost, st));
    SILI_HIP(hipStreamSynchronize(st));
    F.group_base.ensure((size_t)ng + 1);
    F.group_elem.ensure((size_t)ng + 1);
    F.group_pos.ensure((size_t)ng + 1);
    len.ensure((size_t)ng + 1);
    SILI_HIP(hipMemsetAsync(len.p + ng, 0, 4, st));
    if (ng > 0)
        launch(k_for_group_meta, dim3(nblk(ng)), dim3(TPB), 0, st, (const uint32_t *)F.row_group.p, rows,
               (const uint32_t *)W.elem_start.p, (const int32_t *)cols.p, (int64_t)ng, (uint32_t)G, F.group_base.p,
               F.group_elem.p, len.p);
    launch(k_set_u32, dim3(1), dim3(1), 0, st, F.group_elem.p + ng, (uint32_t)N);
    scan_u32(len.p, F.group_pos.p, (int64_t)ng + 1, temp, st);
    uint32_t total = 0;
    SILI_HIP(hipMemcpyAsync(&total, F.group_pos.p + ng, 4, hipMemcpyDeviceToHost, st));
    SILI_HIP(hipStreamSynchronize(st));
    F.bytes.ensure((size_t)total + 4);
    if (ng > 0)
        launch(k_for_group_write, dim3(nblk((int64_t)ng * G)), dim3(TPB), 0, st, (const uint32_t *)F.group_pos.p,
               (const uint32_t *)F.group_base.p, (const uint32_t *)F.group_elem.p, (const int32_t *)cols.p,
               (int64_t)ng, (uint32_t)G, F.bytes.p);
    SILI_HIP(hipGetLastError());
    SILI_HIP(hipStreamSynchronize(st));
    F.G = G;
    F.ngroups = ng;
    F.nbytes = total;
    F.valid = true;
}

void decode_columns(Layer &L, int32_t *cols, int use_for, hipStream_t st) {
    DScatter &W = L.W;
    if (W.nnz == 0) return;
    if (!use_for) {
        ProfScope ps("uleb", st);
        launch_decode(W.plan(), ScaleView{nullptr, nullptr, 1}, cols, nullptr, nullptr, st);
        return;
    }
    const DFor &F = W.fidx;
    if (!F.valid) throw_error(SILI_ERR_INVALID, "decode from the FOR index: build it first (build_for_index)");
    ProfScope ps("for", st);
    const int64_t nslots = F.ngroups * F.G;
    if (nslots >= (int64_t(1) << 32)) throw_error(SILI_ERR_INVALID, "decode from the FOR index: too many slots");
    const auto *bp = (const uint8_t *)F.bytes.p;
    const auto *gp = (const uint32_t *)F.group_pos.p, *gb = (const uint32_t *)F.group_base.p,
               *ge = (const uint32_t *)F.group_elem.p;
    const dim3 grid(nblk(nslots));
    const dim3 ggrid(nblk(F.ngroups));
    if (use_for == 1) {
        // one lane per slot, the group bytes by coalesced dword loads
        const uint32_t ndw = (uint32_t)(F.bytes.n / 4);
        const int64_t waves = (F.ngroups + 64 / F.G - 1) / (64 / F.G);
        const dim3 wgrid((unsigned)((waves + TPB / 64 - 1) / (TPB / 64)));
        switch (F.G) {
            case 8: launch(k_for_decode_wave<8>, wgrid, dim3(TPB), 0, st, bp, ndw, gp, gb, ge, (uint32_t)F.ngroups, cols); break;
            case 16: launch(k_for_decode_wave<16>, wgrid, dim3(TPB), 0, st, bp, ndw, gp, gb, ge, (uint32_t)F.ngroups, cols); break;
            case 32: launch(k_for_decode_wave<32>, wgrid, dim3(TPB), 0, st, bp, ndw, gp, gb, ge, (uint32_t)F.ngroups, cols); break;
            default: launch(k_for_decode_wave<64>, wgrid, dim3(TPB), 0, st, bp, ndw, gp, gb, ge, (uint32_t)F.ngroups, cols); break;
        }
        SILI_HIP(hipGetLastError());
        return;
    }
    // use_for == 2: one thread per group (G 8, 16) or per slot with byte loads
    switch (F.G) {
        case 8: launch(k_for_decode_tg<8>, ggrid, dim3(TPB), 0, st, bp, gp, gb, ge, (uint32_t)F.ngroups, cols); break;
        case 16: launch(k_for_decode_tg<16>, ggrid, dim3(TPB), 0, st, bp, gp, gb, ge, (uint32_t)F.ngroups, cols); break;
        case 32: launch(k_for_decode<32>, grid, dim3(TPB), 0, st, bp, gp, gb, ge, (uint32_t)nslots, cols); break;
        default: launch(k_for_decode<64>, grid, dim3(TPB), 0, st, bp, gp, gb, ge, (uint32_t)nslots, cols); break;
    }
    SILI_HIP(hipGetLastError());
}

}  // namespace sili
