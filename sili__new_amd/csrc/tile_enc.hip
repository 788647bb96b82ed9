// tile_enc.hip -- the reference's block4 tile encoding (block4.hpp:332-388,
// 1016-1031): which tiles its Block4Store holds sparse-packed
// (tile_is_sparse), kept per canonical tile as its operations would set it,
// and the stored bytes for export.  The device always computes on the dense
// 16-byte tiles; this is the format of record for parity and exports.
//
// The encoding follows the reference's rules: a tile is (re-)encoded by its
// live count (sparse iff live <= switch_point) when a load writes it, when it
// is promoted or receives an insert (maybe_compress, delta_csr_memory.hpp:
// 656,698), and when an optimizer update rewrites it (the dense update every
// tile, linear_disldo.hpp:984-1000,1839-1856; the sparse-gradient update the
// tiles with a nonzero dy in one of their columns, sisldo_ops.hpp:945-1033).
// A removal zeroes a slot in place: a dense tile stays dense.
#include "../../include/sili_hip.h"
#include "layer.hpp"
#include "wave.hpp"

#include <cstring>  // host memset, needed before rocprim's headers

#include <rocprim/rocprim.hpp>

namespace sili {

namespace {

constexpr unsigned TPB = 256;
inline unsigned nblk(int64_t n) { return (unsigned)((n + TPB - 1) / TPB); }

__device__ __forceinline__ uint32_t live_of(const uint8_t *t) {
    const uint4 v = *reinterpret_cast<const uint4 *>(t);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    uint32_t n = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int b = 0; b < 4; ++b) n += ((w[i] >> (8 * b)) & 0xFFu) != 0u;
    return n;
}

__global__ void k_tile_reencode(const uint8_t *__restrict__ tiles, int64_t n, uint32_t sp,
                                const uint8_t *__restrict__ dirty, uint8_t *__restrict__ flags) {
    const int64_t t = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (t >= n || (dirty && !dirty[t])) return;
    flags[t] = live_of(tiles + t * 16) <= sp ? 1u : 0u;
}

// dirty[t]: a nonzero dy (in some batch row) in one of tile t's columns
__global__ void k_tile_dirty(const float *__restrict__ gT, int64_t B, int64_t n_out,
                             const uint32_t *__restrict__ tbc, int64_t n, uint8_t *__restrict__ dirty) {
    const int64_t t = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (t >= n) return;
    bool d = false;
    for (uint32_t lj = 0; lj < 4u && !d; ++lj) {
        const int64_t c = (int64_t)tbc[t] * 4 + lj;
        if (c >= n_out) break;
        const float *col = gT + c * B;
        for (int64_t b = 0; b < B && !d; ++b) d = col[b] != 0.0f;
    }
    dirty[t] = d ? 1u : 0u;
}

// stored length: sparse 1 + ceil(live/2) + live (block4.hpp:343-345), dense 16
__global__ void k_tile_len(const uint8_t *__restrict__ tiles, const uint8_t *__restrict__ flags, int64_t n,
                           uint32_t *__restrict__ len, unsigned long long *__restrict__ live_total) {
    const int64_t t = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (t >= n) return;
    const uint32_t live = live_of(tiles + t * 16);
    len[t] = flags[t] ? 1u + (live + 1u) / 2u + live : 16u;
    atomicAdd(live_total, (unsigned long long)live);
}

// block4_sparse_pack (block4.hpp:364-383): [count][positions, even index in
// the high nibble][values], slots ascending; dense tiles are copied.
__global__ void k_tile_pack(const uint8_t *__restrict__ tiles, const uint8_t *__restrict__ flags, int64_t n,
                            const uint32_t *__restrict__ pos, uint8_t *__restrict__ out) {
    const int64_t t = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (t >= n) return;
    const uint8_t *src = tiles + t * 16;
    uint8_t *dst = out + pos[t];
    if (!flags[t]) {
        for (int s = 0; s < 16; ++s) dst[s] = src[s];
        return;
    }
    uint32_t cnt = live_of(src);
    dst[0] = (uint8_t)cnt;
    const uint32_t nib = (cnt + 1u) / 2u;
    for (uint32_t k = 0; k < nib; ++k) dst[1 + k] = 0;
    uint32_t i = 0;
    for (uint32_t s = 0; s < 16u; ++s) {
        if (!src[s]) continue;
        uint8_t &b = dst[1 + i / 2u];
        b = (i % 2u == 0u) ? (uint8_t)((b & 0x0Fu) | (s << 4)) : (uint8_t)((b & 0xF0u) | s);
        dst[1 + nib + i] = src[s];
        ++i;
    }
}

}  // namespace

void tiles_reencode(Layer &L, const uint8_t *dirty, hipStream_t st) {
    const int64_t n = L.B4.ntiles;
    if (n == 0) return;
    L.B4.sparse.ensure((size_t)n + 1);
    launch(k_tile_reencode, dim3(nblk(n)), dim3(TPB), 0, st, (const uint8_t *)L.B4.tiles.p, n, L.switch_point, dirty,
           L.B4.sparse.p);
    SILI_HIP(hipGetLastError());
}

void tiles_reencode_sparse_update(Layer &L, const float *gT, int64_t B, hipStream_t st) {
    const int64_t n = L.B4.ntiles;
    if (n == 0) return;
    DevBuf<uint32_t> br, bc;
    DevBuf<uint8_t> dirty;
    br.ensure((size_t)n);
    bc.ensure((size_t)n);
    dirty.ensure((size_t)n);
    launch_decode_b4(L.B4.plan(), br.p, bc.p, st);
    launch(k_tile_dirty, dim3(nblk(n)), dim3(TPB), 0, st, gT, B, L.n_out, (const uint32_t *)bc.p, n, dirty.p);
    tiles_reencode(L, dirty.p, st);
    SILI_HIP(hipStreamSynchronize(st));
}

PackedTiles export_tiles_packed(Layer &L) {
    PackedTiles out;
    const int64_t n = L.B4.ntiles, brows = (L.n_in + 3) / 4;
    hipStream_t st = L.stream;
    out.row_start.assign((size_t)brows + 1, 0);
    if (n == 0) return out;
    DevBuf<uint32_t> len, pos;
    DevBuf<unsigned long long> live;
    DevBuf<uint8_t> temp, bytes;
    len.ensure((size_t)n + 1);
    pos.ensure((size_t)n + 1);
    live.ensure(1);
    SILI_HIP(hipMemsetAsync(live.p, 0, sizeof(unsigned long long), st));
    SILI_HIP(hipMemsetAsync(len.p + n, 0, 4, st));
    launch(k_tile_len, dim3(nblk(n)), dim3(TPB), 0, st, (const uint8_t *)L.B4.tiles.p, (const uint8_t *)L.B4.sparse.p,
           n, len.p, live.p);
    size_t tb = 0;
    SILI_HIP(rocprim::exclusive_scan(nullptr, tb, len.p, pos.p, uint32_t(0), (size_t)n + 1, rocprim::plus<uint32_t>(), st));
    temp.ensure(tb + 16);
    SILI_HIP(rocprim::exclusive_scan(temp.p, tb, len.p, pos.p, uint32_t(0), (size_t)n + 1, rocprim::plus<uint32_t>(), st));
    uint32_t total = 0;
    SILI_HIP(hipMemcpyAsync(&total, pos.p + n, 4, hipMemcpyDeviceToHost, st));
    SILI_HIP(hipStreamSynchronize(st));
    bytes.ensure((size_t)total + 16);
    launch(k_tile_pack, dim3(nblk(n)), dim3(TPB), 0, st, (const uint8_t *)L.B4.tiles.p, (const uint8_t *)L.B4.sparse.p,
           n, (const uint32_t *)pos.p, bytes.p);
    SILI_HIP(hipGetLastError());
    out.flags.resize((size_t)n);
    out.bytes.resize(total);
    std::vector<uint32_t> hpos((size_t)n + 1), tstart((size_t)brows + 1);
    unsigned long long hlive = 0;
    SILI_HIP(hipMemcpyAsync(out.flags.data(), L.B4.sparse.p, (size_t)n, hipMemcpyDeviceToHost, st));
    if (total) SILI_HIP(hipMemcpyAsync(out.bytes.data(), bytes.p, total, hipMemcpyDeviceToHost, st));
    SILI_HIP(hipMemcpyAsync(hpos.data(), pos.p, hpos.size() * 4, hipMemcpyDeviceToHost, st));
    SILI_HIP(hipMemcpyAsync(tstart.data(), L.B4.tile_start.p, tstart.size() * 4, hipMemcpyDeviceToHost, st));
    SILI_HIP(hipMemcpyAsync(&hlive, live.p, sizeof(hlive), hipMemcpyDeviceToHost, st));
    SILI_HIP(hipStreamSynchronize(st));
    for (int64_t r = 0; r <= brows; ++r) out.row_start[(size_t)r] = hpos[tstart[(size_t)r]];
    out.live = (int64_t)hlive;
    return out;
}

}  // namespace sili
