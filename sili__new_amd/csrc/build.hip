// build.hip -- device builders for the delta-CSR and block4 stores.
//
// Every store is (re)built on the GPU from row-sorted absolute entries:
// per-entry ULEB128 lengths -> exclusive scan -> byte offsets -> encode, plus
// the segment (decode work item) table.  The transposed shadow used by the
// forward pass is a stable radix sort of the canonical entries by column
// (rocprim), re-encoded the same way.  Load, load_dense_codes and every
// synaptogenesis rebuild go through these routines, so a structure is a pure
// function of its entry set -- the canonical encoding
// (delta_csr_memory.hpp:16-93 + sisldo_ops.hpp:44-96).
#include "layer.hpp"
#include "wave.hpp"

#include <algorithm>
#include <cstring>  // host memset, needed before rocprim's headers

#include <rocprim/rocprim.hpp>

namespace sili {

namespace {

constexpr unsigned TPB = 256;
inline unsigned nblk(int64_t n) { return (unsigned)((n + TPB - 1) / TPB); }

__device__ __forceinline__ uint32_t row_of(const uint32_t *__restrict__ ptrs, int64_t rows, uint32_t i) {
    // largest r with ptrs[r] <= i (ptrs non-decreasing, ptrs[0] = 0)
    int64_t lo = 0, hi = rows - 1;
    while (lo < hi) {
        const int64_t mid = (lo + hi + 1) >> 1;
        if (ptrs[mid] <= i) lo = mid;
        else hi = mid - 1;
    }
    return (uint32_t)lo;
}

// Per entry: ULEB length of its column delta; validates order and range.
__global__ void k_entry_len(const uint32_t *__restrict__ ptrs, int64_t rows, int64_t ncols,
                            const uint32_t *__restrict__ cols, int64_t N,
                            uint64_t *__restrict__ len, uint32_t *__restrict__ rowid,
                            int *__restrict__ bad, uint32_t *__restrict__ n_empty) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i >= N) {
        if (i == N) {  // the scan's last term and the row counters start at zero
            len[N] = 0;
            n_empty[0] = 0u;
            n_empty[1] = 0u;
        }
        return;
    }
    const uint32_t r = row_of(ptrs, rows, (uint32_t)i);
    const uint32_t c = cols[i];
    const bool first = (uint32_t)i == ptrs[r];
    const uint32_t prev = first ? 0u : cols[i - 1];
    if ((int64_t)c >= ncols || (!first && c <= prev)) atomicOr(bad, 1);
    len[i] = uleb_len(c - prev);
    rowid[i] = r;
}

__global__ void k_entry_write(const uint32_t *__restrict__ ptrs, const uint32_t *__restrict__ rowid,
                              const uint32_t *__restrict__ cols, int64_t N,
                              const uint64_t *__restrict__ pos, uint8_t *__restrict__ idx) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i >= N) return;
    const uint32_t r = rowid[i];
    const uint32_t c = cols[i];
    uint32_t v = ((uint32_t)i == ptrs[r]) ? c : c - cols[i - 1];
    uint64_t p = pos[i];
    do {
        uint32_t b = v & 0x7Fu;
        v >>= 7;
        if (v) b |= 0x80u;
        idx[p++] = (uint8_t)b;
    } while (v);
}

// Segments split rows by index bytes: segment j holds the entries whose
// varint starts at row offset [j*W, (j+1)*W), W = seg_bytes - 4, so a segment
// never spans more than seg_bytes bytes and never starts inside a varint.
__device__ __forceinline__ uint32_t seg_count(uint32_t n, uint64_t last_start_rel, uint32_t W, int emit_empty) {
    return n == 0u ? (emit_empty ? 1u : 0u) : (uint32_t)(last_start_rel / W) + 1u;
}

__global__ void k_row_starts(const uint32_t *__restrict__ ptrs, int64_t rows, int64_t N,
                             const uint64_t *__restrict__ pos, uint64_t total,
                             uint32_t *__restrict__ byte_start, uint32_t *__restrict__ elem_start,
                             uint32_t seg_bytes, int emit_empty, uint32_t *__restrict__ segcnt,
                             uint32_t *__restrict__ n_empty, int *__restrict__ flag) {
    const int64_t r = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (r > rows) return;
    const uint32_t e = ptrs[r];
    const uint64_t b0 = ((int64_t)e < N) ? pos[e] : total;
    byte_start[r] = (uint32_t)b0;
    elem_start[r] = e;
    // n_empty[1]: rows that are one work item of at most SHORT_ROW_BYTES
    // index bytes (the short rows the float4 gather packs several to a wave),
    // counted per wave
    bool short_row = false;
    if (r < rows) {
        const uint32_t e1 = ptrs[r + 1], n = e1 - e;
        const uint32_t cnt = seg_count(n, n ? pos[e1 - 1] - pos[e] : 0u, seg_bytes - 4u, emit_empty);
        segcnt[r] = cnt;
        if (n == 0u) atomicAdd(n_empty, 1u);
        const uint64_t b1 = (int64_t)e1 < N ? pos[e1] : total;
        short_row = cnt == 1u && b1 - b0 <= SHORT_ROW_BYTES;
    } else {
        segcnt[rows] = 0u;  // the scan's last term
        *flag = 0;          // the work-item writer's split flag
    }
    const uint64_t sb = __ballot(short_row);
    if (sb != 0ull && (threadIdx.x & 63u) == (uint32_t)__builtin_ctzll(sb)) atomicAdd(n_empty + 1, (uint32_t)__popcll(sb));
}

// first entry in [lo, hi) whose varint starts at or after row offset `off`
__device__ __forceinline__ uint32_t first_at(const uint64_t *__restrict__ pos, uint32_t lo, uint32_t hi,
                                             uint64_t base, uint64_t off) {
    while (lo < hi) {
        const uint32_t mid = lo + ((hi - lo) >> 1);
        if (pos[mid] - base < off) lo = mid + 1u;
        else hi = mid;
    }
    return lo;
}

__global__ void k_seg_write(const uint32_t *__restrict__ ptrs, int64_t rows,
                            const uint32_t *__restrict__ byte_start, const uint32_t *__restrict__ cols,
                            const uint64_t *__restrict__ pos, const uint32_t *__restrict__ segoff,
                            uint32_t seg_bytes, int emit_empty, SegDesc *__restrict__ seg,
                            int *__restrict__ any_split) {
    const int64_t r = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (r >= rows) return;
    const uint32_t e0 = ptrs[r], e1 = ptrs[r + 1];
    const uint32_t n = e1 - e0, W = seg_bytes - 4u;
    const uint64_t base = n ? pos[e0] : 0u;
    const uint32_t cnt = seg_count(n, n ? pos[e1 - 1] - base : 0u, W, emit_empty);
    if (cnt > 1u) atomicOr(any_split, 1);
    uint32_t eb = e0;
    for (uint32_t j = 0; j < cnt; ++j) {
        const bool last = j + 1u == cnt;
        const uint32_t ee = last ? e1 : first_at(pos, eb, e1, base, (uint64_t)(j + 1u) * W);
        SegDesc d;
        d.row = (uint32_t)r;
        d.elem_begin = eb;
        d.elem_end = ee;
        d.byte_begin = (j == 0u) ? byte_start[r] : (uint32_t)pos[eb];
        d.byte_end = last ? byte_start[r + 1] : (uint32_t)pos[ee];
        d.base_col = (eb > e0) ? cols[eb - 1] : 0u;
        d.split = (cnt > 1u ? SEG_SPLIT : 0u) | (j == 0u ? SEG_FIRST : 0u);
        d.pad1 = 0u;
        seg[segoff[r] + j] = d;
        eb = ee;
    }
}

// ptrs[r] = first index i with keys[i] >= r  (keys sorted ascending)
__global__ void k_ptrs_from_sorted(const uint32_t *__restrict__ keys, int64_t N, int64_t rows,
                                   uint32_t *__restrict__ ptrs) {
    const int64_t r = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (r > rows) return;
    int64_t lo = 0, hi = N;
    while (lo < hi) {
        const int64_t mid = (lo + hi) >> 1;
        if ((int64_t)keys[mid] < r) lo = mid + 1;
        else hi = mid;
    }
    ptrs[r] = (uint32_t)lo;
}

__global__ void k_gather_u32(const uint32_t *__restrict__ src, const uint32_t *__restrict__ perm,
                             int64_t N, uint32_t *__restrict__ dst) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i < N) dst[i] = src[perm[i]];
}
__global__ void k_gather_u64(const uint64_t *__restrict__ src, const uint32_t *__restrict__ perm,
                             int64_t N, uint64_t *__restrict__ dst) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i < N) dst[i] = src[perm[i]];
}
__global__ void k_gather_u8(const uint8_t *__restrict__ src, const uint32_t *__restrict__ perm,
                            int64_t N, uint8_t *__restrict__ dst) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i < N) dst[i] = src[perm[i]];
}
__global__ void k_iota(uint32_t *__restrict__ v, int64_t N) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i < N) v[i] = (uint32_t)i;
}

// ---- ordering entries by (major, minor), keys unique --------------------
// A counting pass by major (atomics), an exclusive scan into each major's
// first position, a scatter into the majors' segments (arbitrary order within
// a segment), then each segment ordered by minor: one wave per segment, a
// bitonic network over the wave's lanes (up to 64 entries) or in the wave's
// LDS slice (up to SEGSORT_CAP; at 2048 its 64 KiB blocks left 8 waves per
// CU), a longer segment by one block in global memory.  The order within a
// segment is unique since the keys are, so the result equals a sort of the
// keys.  About six launches where a device radix sort of a few hundred
// thousand keys took about twenty.
constexpr uint32_t SEGSORT_CAP = 512;
constexpr uint32_t SEGSORT_WAVES = 4;
constexpr uint32_t LONG_LDS_CAP = 8192, LONG_MAX_BLOCKS = 65536;

__global__ void k_fill_u32_b(uint32_t *__restrict__ p, int64_t n, uint32_t v) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i < n) p[i] = v;
}

__global__ void k_count_major(const uint32_t *__restrict__ maj, int64_t N, int64_t maj_ext,
                              uint32_t *__restrict__ cnt, int *__restrict__ bad) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i >= N) return;
    const uint32_t m = maj[i];
    if ((int64_t)m >= maj_ext) {
        atomicOr(bad, 1);
        atomicAdd(cnt + maj_ext, 1u);  // kept last, so that perm stays a permutation
        return;
    }
    atomicAdd(cnt + m, 1u);
}

// cnt (the counts) is consumed: each entry takes position ptr[m] + (its
// count after the decrement).  An out-of-range major (flagged by the count)
// goes after every segment, directly into perm.
__global__ void k_scatter_major(const uint32_t *__restrict__ maj, const uint32_t *__restrict__ mnr, int64_t N,
                                int64_t maj_ext, const uint32_t *__restrict__ ptr, uint32_t *__restrict__ cnt,
                                uint32_t *__restrict__ seg_mnr, uint32_t *__restrict__ seg_idx,
                                uint32_t *__restrict__ perm) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i >= N) return;
    const uint32_t m = maj[i];
    if ((int64_t)m >= maj_ext) {
        perm[ptr[maj_ext] + atomicSub(cnt + maj_ext, 1u) - 1u] = (uint32_t)i;
        return;
    }
    const uint32_t p = ptr[m] + atomicSub(cnt + m, 1u) - 1u;
    seg_mnr[p] = mnr[i];
    seg_idx[p] = (uint32_t)i;
}

// The same two passes with each block's share counted in LDS first, for at
// most MM_BINS majors: one global atomic per (block, major present) instead
// of one per entry, which matters when few majors take many entries each
// (a block4 store's 4096 block columns of ~127 tiles).  Each block takes
// MM_CHUNK consecutive entries, MM_PER = MM_CHUNK / 256 per thread.
constexpr uint32_t MM_BINS = 8192, MM_PER = 32, MM_CHUNK = 256 * MM_PER;

__global__ __launch_bounds__(256) void k_count_major_lds(const uint32_t *__restrict__ maj, int64_t N,
                                                         int64_t maj_ext, uint32_t *__restrict__ cnt,
                                                         int *__restrict__ bad) {
    __shared__ uint32_t h[MM_BINS + 1];  // [maj_ext]: out-of-range majors
    for (uint32_t i = threadIdx.x; i <= (uint32_t)maj_ext; i += 256u) h[i] = 0u;
    __syncthreads();
    const int64_t e0 = (int64_t)blockIdx.x * MM_CHUNK + threadIdx.x;
#pragma unroll 4
    for (uint32_t k = 0; k < MM_PER; ++k) {
        const int64_t e = e0 + (int64_t)k * 256;
        if (e < N) {
            const uint32_t m = maj[e];
            if ((int64_t)m >= maj_ext) atomicOr(bad, 1);
            atomicAdd(&h[(int64_t)m < maj_ext ? m : (uint32_t)maj_ext], 1u);
        }
    }
    __syncthreads();
    for (uint32_t i = threadIdx.x; i <= (uint32_t)maj_ext; i += 256u)
        if (h[i]) atomicAdd(cnt + i, h[i]);
}

// Positions: an entry's rank among its block's entries of the same major (LDS
// atomics), plus the block's base in the major's segment, taken from cnt (the
// counts, consumed) by one atomic per major present.
__global__ __launch_bounds__(256) void k_scatter_major_lds(const uint32_t *__restrict__ maj,
                                                           const uint32_t *__restrict__ mnr, int64_t N,
                                                           int64_t maj_ext, const uint32_t *__restrict__ ptr,
                                                           uint32_t *__restrict__ cnt, uint32_t *__restrict__ seg_mnr,
                                                           uint32_t *__restrict__ seg_idx, uint32_t *__restrict__ perm) {
    __shared__ uint32_t h[MM_BINS + 1];  // [maj_ext]: out-of-range majors, placed last
    for (uint32_t i = threadIdx.x; i <= (uint32_t)maj_ext; i += 256u) h[i] = 0u;
    __syncthreads();
    const int64_t e0 = (int64_t)blockIdx.x * MM_CHUNK + threadIdx.x;
    uint32_t rk[MM_PER];
#pragma unroll
    for (uint32_t k = 0; k < MM_PER; ++k) {
        const int64_t e = e0 + (int64_t)k * 256;
        rk[k] = 0u;
        if (e < N) {
            const uint32_t m = maj[e];
            rk[k] = atomicAdd(&h[(int64_t)m < maj_ext ? m : (uint32_t)maj_ext], 1u);
        }
    }
    __syncthreads();
    // h[m] becomes the block's first position in major m's segment
    for (uint32_t i = threadIdx.x; i <= (uint32_t)maj_ext; i += 256u) {
        const uint32_t c = h[i];
        if (c) h[i] = ptr[i] + atomicSub(cnt + i, c) - c;
    }
    __syncthreads();
#pragma unroll
    for (uint32_t k = 0; k < MM_PER; ++k) {
        const int64_t e = e0 + (int64_t)k * 256;
        if (e < N) {
            const uint32_t m = maj[e];
            if ((int64_t)m < maj_ext) {
                const uint32_t p = h[m] + rk[k];
                seg_mnr[p] = mnr[e];
                seg_idx[p] = (uint32_t)e;
            } else {
                perm[h[maj_ext] + rk[k]] = (uint32_t)e;
            }
        }
    }
}

// perm[p] for every position of segment m (one wave per segment); a segment
// longer than SEGSORT_CAP is listed for k_seg_sort_long.
__global__ __launch_bounds__(SEGSORT_WAVES * 64) void k_seg_sort_minor(const uint32_t *__restrict__ ptr, int64_t nseg,
                                                                      const uint32_t *__restrict__ seg_mnr,
                                                                      const uint32_t *__restrict__ seg_idx,
                                                                      uint32_t *__restrict__ perm,
                                                                      uint32_t *__restrict__ n_long,
                                                                      uint32_t *__restrict__ longs) {
    __shared__ uint2 s[SEGSORT_WAVES][SEGSORT_CAP];
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const int64_t m = (int64_t)blockIdx.x * SEGSORT_WAVES + wave;
    if (m >= nseg) return;
    const uint32_t b = ptr[m], len = ptr[m + 1] - b;
    if (len <= 1u) {
        if (len == 1u && lane == 0) perm[b] = seg_idx[b];
        return;
    }
    if (len <= 64u) {
        // bitonic network over the lanes; padding sorts last (minor < 2^32 - 1)
        uint32_t key = lane < len ? seg_mnr[b + lane] : 0xFFFFFFFFu;
        uint32_t idx = lane < len ? seg_idx[b + lane] : 0u;
        for (uint32_t k = 2; k <= 64u; k <<= 1)
            for (uint32_t j = k >> 1; j > 0; j >>= 1) {
                const uint32_t ok = (uint32_t)__shfl_xor((int)key, (int)j, 64);
                const uint32_t oi = (uint32_t)__shfl_xor((int)idx, (int)j, 64);
                const bool up = (lane & k) == 0u, lower = (lane & j) == 0u;
                if (lower == up ? ok < key : ok > key) {
                    key = ok;
                    idx = oi;
                }
            }
        if (lane < len) perm[b + lane] = idx;
        return;
    }
    if (len > SEGSORT_CAP) {
        if (lane == 0) longs[atomicAdd(n_long, 1u)] = (uint32_t)m;
        return;
    }
    uint32_t n2 = 128;
    while (n2 < len) n2 <<= 1;
    uint2 *t = s[wave];
    for (uint32_t q = lane; q < n2; q += 64u)
        t[q] = q < len ? make_uint2(seg_mnr[b + q], seg_idx[b + q]) : make_uint2(0xFFFFFFFFu, 0u);
    wave_lds_sync();
    for (uint32_t k = 2; k <= n2; k <<= 1)
        for (uint32_t j = k >> 1; j > 0; j >>= 1) {
            for (uint32_t q = lane; q < n2 / 2u; q += 64u) {
                const uint32_t lo = (q / j) * 2u * j + (q % j), hi = lo + j;
                const bool up = (lo & k) == 0u;
                const uint2 x = t[lo], y = t[hi];
                if (up ? x.x > y.x : x.x < y.x) {
                    t[lo] = y;
                    t[hi] = x;
                }
            }
            wave_lds_sync();
        }
    for (uint32_t q = lane; q < len; q += 64u) perm[b + q] = t[q].y;
}

// The listed long segments, one block each: up to LONG_LDS_CAP entries by a
// bitonic network in the block's LDS; beyond, in place in seg_mnr /
// seg_idx by a bitonic network whose comparators all put the smaller minor
// first (each merge starts by comparing mirrored positions), so positions at
// or past the segment's end act as +infinity and their comparators are
// skipped; then perm.  Minors are unique within a segment.
__global__ __launch_bounds__(256) void k_seg_sort_long(const uint32_t *__restrict__ ptr,
                                                       const uint32_t *__restrict__ n_long,
                                                       const uint32_t *__restrict__ longs, uint32_t *seg_mnr,
                                                       uint32_t *seg_idx, uint32_t *__restrict__ perm) {
    __shared__ uint2 t[LONG_LDS_CAP];
    const uint32_t nl = *n_long;
    for (uint32_t q = blockIdx.x; q < nl; q += gridDim.x) {
        const uint32_t m = longs[q], b = ptr[m], len = ptr[m + 1] - b;
        uint32_t *mn = seg_mnr + b, *ix = seg_idx + b;
        uint32_t n2 = 1;
        while (n2 < len) n2 <<= 1;
        if (len <= LONG_LDS_CAP) {
            // the block's LDS: a plain bitonic network, padding sorting last
            for (uint32_t i = threadIdx.x; i < n2; i += 256u)
                t[i] = i < len ? make_uint2(mn[i], ix[i]) : make_uint2(0xFFFFFFFFu, 0u);
            __syncthreads();
            for (uint32_t k = 2; k <= n2; k <<= 1)
                for (uint32_t j = k >> 1; j > 0; j >>= 1) {
                    for (uint32_t i = threadIdx.x; i < n2 / 2u; i += 256u) {
                        const uint32_t lo = (i / j) * 2u * j + (i % j), hi = lo + j;
                        const bool up = (lo & k) == 0u;
                        const uint2 x = t[lo], y = t[hi];
                        if (up ? x.x > y.x : x.x < y.x) {
                            t[lo] = y;
                            t[hi] = x;
                        }
                    }
                    __syncthreads();
                }
            for (uint32_t i = threadIdx.x; i < len; i += 256u) perm[b + i] = t[i].y;
            __syncthreads();
            continue;
        }
        for (uint32_t k = 2; k <= n2; k <<= 1)
            for (uint32_t j = k >> 1; j > 0; j >>= 1) {
                for (uint32_t t = threadIdx.x; t < n2 / 2u; t += 256u) {
                    const uint32_t lo = (t / j) * 2u * j + (t % j);
                    const uint32_t hi = j == (k >> 1) ? (lo / k) * k + (k - 1u) - (lo % k) : lo + j;
                    if (hi < len) {
                        const uint32_t a = mn[lo], c = mn[hi];
                        if (a > c) {
                            const uint32_t ia = ix[lo];
                            mn[lo] = c;
                            mn[hi] = a;
                            ix[lo] = ix[hi];
                            ix[hi] = ia;
                        }
                    }
                }
                __syncthreads();
            }
        for (uint32_t t = threadIdx.x; t < len; t += 256u) perm[b + t] = ix[t];
        __syncthreads();
    }
}

// Block4: key = major * minor_extent + minor.
__global__ void k_tile_keys(const uint32_t *__restrict__ major, const uint32_t *__restrict__ minor,
                            int64_t N, uint64_t minor_extent, int64_t major_extent,
                            uint64_t *__restrict__ key, int *__restrict__ bad) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i >= N) return;
    if ((int64_t)major[i] >= major_extent || (uint64_t)minor[i] >= minor_extent) atomicOr(bad, 1);
    key[i] = (uint64_t)major[i] * minor_extent + minor[i];
}
__global__ void k_split_keys(const uint64_t *__restrict__ key, int64_t N, uint64_t minor_extent,
                             uint32_t *__restrict__ major, uint32_t *__restrict__ minor,
                             int *__restrict__ bad) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i >= N) return;
    const uint64_t k = key[i];
    if (i > 0 && key[i - 1] == k) atomicOr(bad, 2);  // duplicate tile
    if (i > 0 && key[i - 1] > k) atomicOr(bad, 4);   // merged runs out of order
    major[i] = (uint32_t)(k / minor_extent);
    minor[i] = (uint32_t)(k % minor_extent);
}
// dst tile i = src tile perm[i], optionally 4x4-transposed (slot lj*4+li <-> li*4+lj).
// inv[perm[i]] = i
__global__ void k_inv_perm(const uint32_t *__restrict__ perm, int64_t N, uint32_t *__restrict__ inv) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i < N) inv[perm[i]] = (uint32_t)i;
}
// out[j] = inv[perm[j]]
__global__ void k_compose_perm(const uint32_t *__restrict__ perm, const uint32_t *__restrict__ inv, int64_t N,
                               uint32_t *__restrict__ out) {
    const int64_t j = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (j < N) out[j] = inv[perm[j]];
}

__global__ void k_gather_tiles(const uint8_t *__restrict__ src, const uint32_t *__restrict__ perm,
                               int64_t N, int transpose, uint8_t *__restrict__ dst) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i >= N) return;
    const uint4 v = *reinterpret_cast<const uint4 *>(src + (size_t)perm[i] * 16u);
    if (!transpose) {
        *reinterpret_cast<uint4 *>(dst + (size_t)i * 16u) = v;
        return;
    }
    uint8_t in[16], out[16];
    *reinterpret_cast<uint4 *>(in) = v;
#pragma unroll
    for (int li = 0; li < 4; ++li)
#pragma unroll
        for (int lj = 0; lj < 4; ++lj) out[li * 4 + lj] = in[lj * 4 + li];
    *reinterpret_cast<uint4 *>(dst + (size_t)i * 16u) = *reinterpret_cast<uint4 *>(out);
}

// Scattered weight code 8 (NaN) present?
__global__ void k_scan_nan_codes(const uint8_t *__restrict__ v, int64_t N, int hi_nibble,
                                 int *__restrict__ flag) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i >= N) return;
    const uint32_t code = hi_nibble ? ((uint32_t)v[i] >> 4) : ((uint32_t)v[i] & 0xFu);
    if (code == 8u) atomicOr(flag, 1);
}

void check_flag(Layer &L, int *d_flag, const char *what) {
    int h = 0;
    ReadBack rb(L);
    rb.add(&h, d_flag, sizeof(int));
    rb.wait();
    if (h & 4) throw_error(3, std::string(what) + ": merged tile runs out of order (internal error)");
    if (h) throw_error(1, std::string(what) + (h & 2 ? ": duplicate entries" : ": malformed input (unsorted, duplicate or out-of-range index)"));
}

void zero_flag(Layer &L) {
    L.scratch.flag.ensure(4, 0);
    SILI_HIP(hipMemsetAsync(L.scratch.flag.p, 0, 4 * sizeof(int), L.stream));
}

// Encode rows: ptrs[rows+1] (device u32), cols[N].  Fills byte_start,
// elem_start, idx, seg of a store.
struct Encoded {
    int64_t nbytes = 0, nseg = 0;
    bool has_split = false;
    int64_t n_split = 0;
    int64_t n_empty_rows = 0;
    int64_t n_short = 0;  // rows that are one work item of <= SHORT_ROW_BYTES index bytes
};

__global__ void k_split_flags(const uint32_t *__restrict__ segcnt, int64_t rows, uint32_t *__restrict__ flag) {
    const int64_t r = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (r <= rows) flag[r] = (r < rows && segcnt[r] > 1u) ? 1u : 0u;
}
__global__ void k_split_list(const uint32_t *__restrict__ flag, const uint32_t *__restrict__ pos, int64_t rows,
                             uint32_t *__restrict__ list) {
    const int64_t r = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (r < rows && flag[r]) list[pos[r]] = (uint32_t)r;
}

Encoded encode_rows(Layer &L, int64_t rows, int64_t ncols, int64_t N, const uint32_t *d_ptrs,
                    const uint32_t *d_cols, uint32_t seg_len, bool emit_empty,
                    DevBuf<uint32_t> &byte_start, DevBuf<uint32_t> &elem_start, DevBuf<uint8_t> &idx,
                    DevBuf<SegDesc> &seg, const char *what, DevBuf<uint32_t> *split_rows = nullptr) {
    // Two host round trips: the index stream's size (its buffer is allocated
    // to it) with the input check, then every count at the end.  The work
    // items and the split-row list are allocated to their bounds (a row of
    // b index bytes holds at most b / (seg_len - 4) + 1 work items).
    Encoded out;
    hipStream_t st = L.stream;
    TmpBuf<uint64_t> len(L, SILI_TMPKEY(len)), pos(L, SILI_TMPKEY(pos));
    TmpBuf<uint32_t> rowid(L, SILI_TMPKEY(rowid)), segcnt(L, SILI_TMPKEY(segcnt)), segoff(L, SILI_TMPKEY(segoff));
    len.ensure((size_t)N + 1);
    pos.ensure((size_t)N + 1);
    rowid.ensure((size_t)N + 1);
    zero_flag(L);
    TmpBuf<uint32_t> n_empty(L, SILI_TMPKEY(n_empty));
    n_empty.ensure(2);
    // len[N] and n_empty are zeroed by the length kernel's thread N
    launch(k_entry_len, dim3(nblk(N + 1)), dim3(TPB), 0, st, d_ptrs, rows, ncols, d_cols, N, len.p, rowid.p,
           L.scratch.flag.p, n_empty.p);
    SILI_HIP(hipGetLastError());
    // pos = exclusive scan of len (N+1 entries: pos[N] = total)
    device_exclusive_scan_u64(L, len.p, pos.p, N + 1);
    uint64_t total = 0;
    int bad = 0;
    ReadBack rb(L);
    rb.add(&total, pos.p + N, sizeof(uint64_t));
    rb.add(&bad, L.scratch.flag.p, sizeof(int));
    rb.wait();
    if (bad) throw_error(1, std::string(what) + (bad & 2 ? ": duplicate entries" : ": malformed input (unsorted, duplicate or out-of-range index)"));
    if (total >= (1ull << 32)) throw_error(2, std::string(what) + ": index stream exceeds 4 GiB");
    out.nbytes = (int64_t)total;
    idx.ensure((size_t)total + 64);
    byte_start.ensure((size_t)rows + 1);
    elem_start.ensure((size_t)rows + 1);
    segcnt.ensure((size_t)rows + 1);
    segoff.ensure((size_t)rows + 1);
    if (N > 0) {
        launch(k_entry_write, dim3(nblk(N)), dim3(TPB), 0, st, d_ptrs, rowid.p, d_cols, N,
                           pos.p, idx.p);
        SILI_HIP(hipGetLastError());
    }
    // segcnt[rows] and the split flag are zeroed by the row kernel's thread rows
    launch(k_row_starts, dim3(nblk(rows + 1)), dim3(TPB), 0, st, d_ptrs, rows, N, pos.p,
                       total, byte_start.p, elem_start.p, seg_len, emit_empty ? 1 : 0, segcnt.p, n_empty.p,
                       L.scratch.flag.p);
    SILI_HIP(hipGetLastError());
    device_exclusive_scan_u32(L, segcnt.p, segoff.p, rows + 1);
    const int64_t seg_max = rows + (int64_t)(total / (seg_len - 4u)) + 1;
    seg.ensure((size_t)seg_max + 1);
    if (rows > 0) {
        launch(k_seg_write, dim3(nblk(rows)), dim3(TPB), 0, st, d_ptrs, rows, byte_start.p,
                           d_cols, pos.p, segoff.p, seg_len, emit_empty ? 1 : 0, seg.p, L.scratch.flag.p);
        SILI_HIP(hipGetLastError());
    }
    TmpBuf<uint32_t> fpos(L, SILI_TMPKEY(fpos));
    if (split_rows) {
        // the rows that span several work items (their outputs need zeroing
        // before the atomically combined partial sums), listed whether or not
        // there are any
        TmpBuf<uint32_t> flag(L, SILI_TMPKEY(flag));
        flag.ensure((size_t)rows + 1);
        fpos.ensure((size_t)rows + 1);
        launch(k_split_flags, dim3(nblk(rows + 1)), dim3(TPB), 0, st, (const uint32_t *)segcnt.p, rows, flag.p);
        SILI_HIP(hipGetLastError());
        device_exclusive_scan_u32(L, flag.p, fpos.p, rows + 1);
        split_rows->ensure((size_t)rows + 1);
        launch(k_split_list, dim3(nblk(rows)), dim3(TPB), 0, st, (const uint32_t *)flag.p, (const uint32_t *)fpos.p,
               rows, split_rows->p);
        SILI_HIP(hipGetLastError());
    }
    uint32_t nseg = 0, empty = 0, ns = 0, nshort = 0;
    int split = 0;
    rb.add(&nseg, segoff.p + rows, sizeof(uint32_t));
    rb.add(&empty, n_empty.p, sizeof(uint32_t));
    rb.add(&nshort, n_empty.p + 1, sizeof(uint32_t));
    rb.add(&split, L.scratch.flag.p, sizeof(int));
    if (split_rows) rb.add(&ns, fpos.p + rows, sizeof(uint32_t));
    rb.wait();
    if ((int64_t)nseg > seg_max) throw_error(3, std::string(what) + ": work items exceed their bound (internal error)");
    out.nseg = nseg;
    out.n_empty_rows = empty;
    out.n_short = nshort;
    out.has_split = split != 0;
    if (out.has_split && split_rows) out.n_split = ns;
    return out;
}

}  // namespace

// ---- rocprim wrappers -------------------------------------------------------
void device_exclusive_scan_u64(Layer &L, const uint64_t *in, uint64_t *out, int64_t n) {
    size_t bytes = 0;
    SILI_HIP(rocprim::exclusive_scan(nullptr, bytes, in, out, uint64_t(0), (size_t)n,
                                     rocprim::plus<uint64_t>(), L.stream));
    L.scratch.temp_for(bytes);
    SILI_HIP(rocprim::exclusive_scan(L.scratch.temp.p, bytes, in, out, uint64_t(0), (size_t)n,
                                     rocprim::plus<uint64_t>(), L.stream));
}
// Lane i * 64 + b copies byte b of value i into the pinned buffer (kernels
// write pinned host memory directly; the wait that follows makes it visible).
__global__ __launch_bounds__(512) void k_readback(ReadBackSrc a, uint8_t *__restrict__ dst) {
    const int i = (int)(threadIdx.x >> 6), b = (int)(threadIdx.x & 63u);
    if (i < a.n && (uint32_t)b < a.bytes[i]) dst[64 * i + b] = static_cast<const uint8_t *>(a.src[i])[b];
}

void readback_launch(Layer &L, const ReadBackSrc &a) {
    launch(k_readback, dim3(1), dim3(512), 0, L.stream, a, L.pin_read.h);
    SILI_HIP(hipGetLastError());
}

void device_exclusive_scan_u32(Layer &L, const uint32_t *in, uint32_t *out, int64_t n) {
    size_t bytes = 0;
    SILI_HIP(rocprim::exclusive_scan(nullptr, bytes, in, out, uint32_t(0), (size_t)n,
                                     rocprim::plus<uint32_t>(), L.stream));
    L.scratch.temp_for(bytes);
    SILI_HIP(rocprim::exclusive_scan(L.scratch.temp.p, bytes, in, out, uint32_t(0), (size_t)n,
                                     rocprim::plus<uint32_t>(), L.stream));
}
void device_sort_pairs_u32(Layer &L, const uint32_t *kin, uint32_t *kout, const uint32_t *vin,
                           uint32_t *vout, int64_t n, int bits) {
    size_t bytes = 0;
    SILI_HIP(rocprim::radix_sort_pairs(nullptr, bytes, kin, kout, vin, vout, (size_t)n, 0u,
                                       (unsigned)bits, L.stream));
    L.scratch.temp_for(bytes);
    SILI_HIP(rocprim::radix_sort_pairs(L.scratch.temp.p, bytes, kin, kout, vin, vout, (size_t)n, 0u,
                                       (unsigned)bits, L.stream));
}
void device_sort_pairs_u64(Layer &L, const uint64_t *kin, uint64_t *kout, const uint32_t *vin,
                           uint32_t *vout, int64_t n, int bits) {
    size_t bytes = 0;
    SILI_HIP(rocprim::radix_sort_pairs(nullptr, bytes, kin, kout, vin, vout, (size_t)n, 0u,
                                       (unsigned)bits, L.stream));
    L.scratch.temp_for(bytes);
    SILI_HIP(rocprim::radix_sort_pairs(L.scratch.temp.p, bytes, kin, kout, vin, vout, (size_t)n, 0u,
                                       (unsigned)bits, L.stream));
}

// Two sorted runs of (key, value) pairs merged into one sorted sequence.
static void device_merge_pairs_u64(Layer &L, const uint64_t *k1, const uint64_t *k2, uint64_t *kout,
                                   const uint32_t *v1, const uint32_t *v2, uint32_t *vout, int64_t n1,
                                   int64_t n2) {
    size_t bytes = 0;
    SILI_HIP(rocprim::merge(nullptr, bytes, k1, k2, kout, v1, v2, vout, (size_t)n1, (size_t)n2,
                            rocprim::less<uint64_t>(), L.stream));
    void *temp = L.scratch.temp_for(bytes);
    SILI_HIP(rocprim::merge(temp, bytes, k1, k2, kout, v1, v2, vout, (size_t)n1, (size_t)n2,
                            rocprim::less<uint64_t>(), L.stream));
}

// perm[p]: the entry at position p when the N entries are ordered by
// (major, minor) (keys unique); ptr[0, maj_ext]: each major's first position
// (ptr[maj_ext] = N).  A major out of range sets *bad |= 1 (its entries go
// last, so perm is a permutation whatever the input).  *bad is read back here
// and, if set, raised as `what`'s malformed-input error -- one wait on the
// stream -- except in a build from the layer's own arrays
// (L.trusted_build), which queues everything and returns at once.
static void sort_major_minor(Layer &L, const uint32_t *maj, const uint32_t *mnr, int64_t N, int64_t maj_ext,
                             uint32_t *perm, uint32_t *ptr, int *bad, const char *what) {
    hipStream_t st = L.stream;
    TmpBuf<uint32_t> cnt(L, SILI_TMPKEY(mm_cnt)), smn(L, SILI_TMPKEY(mm_mnr)), sidx(L, SILI_TMPKEY(mm_idx)),
        longs(L, SILI_TMPKEY(mm_longs));
    cnt.ensure((size_t)maj_ext + 2);  // [maj_ext + 1]: the long-segment count
    smn.ensure((size_t)N + 1);
    sidx.ensure((size_t)N + 1);
    longs.ensure((size_t)(N / (SEGSORT_CAP + 1) + 1));
    launch(k_fill_u32_b, dim3(nblk(maj_ext + 2)), dim3(TPB), 0, st, cnt.p, maj_ext + 2, 0u);
    const bool lds = maj_ext <= (int64_t)MM_BINS;
    const unsigned cgrid = (unsigned)((N + MM_CHUNK - 1) / MM_CHUNK);
    if (N > 0 && lds) launch(k_count_major_lds, dim3(cgrid), dim3(256), 0, st, maj, N, maj_ext, cnt.p, bad);
    else if (N > 0) launch(k_count_major, dim3(nblk(N)), dim3(TPB), 0, st, maj, N, maj_ext, cnt.p, bad);
    device_exclusive_scan_u32(L, cnt.p, ptr, maj_ext + 1);
    if (N > 0) {
        if (lds)
            launch(k_scatter_major_lds, dim3(cgrid), dim3(256), 0, st, maj, mnr, N, maj_ext, (const uint32_t *)ptr,
                   cnt.p, smn.p, sidx.p, perm);
        else
            launch(k_scatter_major, dim3(nblk(N)), dim3(TPB), 0, st, maj, mnr, N, maj_ext, (const uint32_t *)ptr,
                   cnt.p, smn.p, sidx.p, perm);
        launch(k_seg_sort_minor, dim3((unsigned)((maj_ext + SEGSORT_WAVES - 1) / SEGSORT_WAVES)),
               dim3(SEGSORT_WAVES * 64), 0, st, (const uint32_t *)ptr, maj_ext, (const uint32_t *)smn.p,
               (const uint32_t *)sidx.p, perm, cnt.p + maj_ext + 1, longs.p);
        // (one block per possible long segment, up to LONG_MAX_BLOCKS; blocks
        // past the listed count return at once)
        const unsigned lgrid = (unsigned)std::min<int64_t>(N / (SEGSORT_CAP + 1) + 1, LONG_MAX_BLOCKS);
        launch(k_seg_sort_long, dim3(lgrid), dim3(256), 0, st, (const uint32_t *)ptr,
               (const uint32_t *)(cnt.p + maj_ext + 1), (const uint32_t *)longs.p, smn.p, sidx.p, perm);
    }
    SILI_HIP(hipGetLastError());
    if (L.trusted_build) return;
    int hb = 0;
    ReadBack rb(L);
    rb.add(&hb, bad, sizeof(int));
    rb.wait();
    if (hb) throw_error(1, std::string(what) + ": malformed input (unsorted, duplicate or out-of-range index)");
}

static int bits_for(uint64_t max_value) {
    int b = 1;
    while (b < 64 && (max_value >> b) != 0) ++b;
    return b;
}

__global__ void k_clear_u32(uint32_t *__restrict__ p, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i < n) p[i] = 0u;
}

// SILI_SPLIT_COMBINE=1 (read when a store is built; default 0): the float4
// gathers combine a split row's work items in item order instead of with
// float atomics, so the rows' sums do not depend on the order in which the
// items finish (bitwise reproducible).  It costs time: on the config-2
// grad-input gather (1594 split rows in 5445 items) 41.5 us against 36.5 us
// with atomics, the combining waves waiting on their write-through stores.
// Buffers: arrival counters (cleared here; each combining launch leaves them
// zero) and one partial-sum slot per work item and batch column, for passes
// of up to 128 columns and at most 16 Mi floats (a store past that, or a
// wider pass, combines with atomics).
void prepare_split_combine(Layer &L, DScatter &s) {
    const int64_t cap = s.nseg * 128;
    if (!s.has_split || s.nseg == 0 || cap > ((int64_t)16 << 20) || env_int("SILI_SPLIT_COMBINE", 0) == 0) {
        s.part_cap = 0;
        return;
    }
    s.part.ensure((size_t)cap, 0);
    s.split_cnt.ensure((size_t)s.rows + 1);
    launch(k_clear_u32, dim3(nblk(s.rows + 1)), dim3(TPB), 0, L.stream, s.split_cnt.p, s.rows + 1);
    SILI_HIP(hipGetLastError());
    s.part_cap = cap;
}

namespace {
// flag[i]: work item i is a whole row of <= SHORT_ROW_BYTES index bytes
// (flag[n] = 0, the scan's last term)
__global__ void k_short_flags(const SegDesc *__restrict__ seg, int64_t n, uint32_t *__restrict__ flag) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i < n) {
        const SegDesc d = seg[i];
        flag[i] = (!(d.split & SEG_SPLIT) && d.byte_end - d.byte_begin <= SHORT_ROW_BYTES) ? 1u : 0u;
    } else if (i == n) {
        flag[n] = 0u;
    }
}
__global__ void k_short_split(const SegDesc *__restrict__ seg, int64_t n, const uint32_t *__restrict__ flag,
                              const uint32_t *__restrict__ pos, SegDesc *__restrict__ sh, SegDesc *__restrict__ lg) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i >= n) return;
    if (flag[i]) sh[pos[i]] = seg[i];
    else lg[i - (int64_t)pos[i]] = seg[i];
}

// Split s's work items into short rows and the others (DScatter::sh_seg),
// once per structure, where a quarter of the items or more are short rows
// (SILI_SHORT_ROWS=0: never).
void ensure_short_rows(Layer &L, DScatter &s) {
    if (s.sh_valid) return;
    s.sh_valid = true;
    s.n_sh = 0;
    s.n_lg = s.nseg;
    if (env_int("SILI_SHORT_ROWS", 1) == 0) return;
    if (s.nseg == 0 || s.n_short_hint < 1024 || s.n_short_hint * 4 < s.nseg) return;
    hipStream_t st = L.stream;
    TmpBuf<uint32_t> flag(L, SILI_TMPKEY(flag)), pos(L, SILI_TMPKEY(pos));
    flag.ensure((size_t)s.nseg + 1);
    pos.ensure((size_t)s.nseg + 1);
    launch(k_short_flags, dim3(nblk(s.nseg + 1)), dim3(TPB), 0, st, (const SegDesc *)s.seg.p, s.nseg, flag.p);
    SILI_HIP(hipGetLastError());
    device_exclusive_scan_u32(L, flag.p, pos.p, s.nseg + 1);
    uint32_t nsh = 0;
    ReadBack rb(L);
    rb.add(&nsh, pos.p + s.nseg, sizeof(uint32_t));
    rb.wait();
    if (nsh < 1024 || (int64_t)nsh * 4 < s.nseg) return;
    s.sh_seg.ensure((size_t)nsh);
    s.lg_seg.ensure((size_t)(s.nseg - nsh) + 1);
    launch(k_short_split, dim3(nblk(s.nseg)), dim3(TPB), 0, st, (const SegDesc *)s.seg.p, s.nseg,
           (const uint32_t *)flag.p, (const uint32_t *)pos.p, s.sh_seg.p, s.lg_seg.p);
    SILI_HIP(hipGetLastError());
    s.n_sh = nsh;
    s.n_lg = s.nseg - nsh;
}
}  // namespace

GatherPlan gather_plan(Layer &L, DScatter &s, int64_t nb) {
    GatherPlan p = s.plan();
    if (nb > 1 && nb <= SHORT_MAX_BATCH && nb % 4 == 0) {
        ensure_short_rows(L, s);
        if (s.n_sh > 0) {
            p.sh_seg = s.sh_seg.p;
            p.n_sh = s.n_sh;
            p.lg_seg = s.lg_seg.p;
            p.n_lg = s.n_lg;
        }
    }
    return p;
}

void build_scattered(Layer &L, DScatter &dst, int64_t rows, int64_t ncols, int64_t N,
                     const uint32_t *d_ptrs, const uint32_t *d_cols, const uint8_t *d_bytes) {
    const Encoded e = encode_rows(L, rows, ncols, N, d_ptrs, d_cols, L.seg_len, true, dst.byte_start,
                                  dst.elem_start, dst.idx, dst.seg, "load_weights", &dst.split_rows);
    dst.n_split = e.n_split;
    dst.stream1.valid = dst.streamK.valid = false;
    dst.fidx.valid = false;
    dst.dcol_valid = false;
    dst.sh_valid = false;
    dst.n_short_hint = e.n_short;
    dst.slc_w = 0;
    dst.stream1.failed = dst.streamK.failed = false;
    dst.cblk.clear();
    dst.cblk_cb = 0;
    dst.rows = rows;
    dst.cols = ncols;
    dst.nnz = N;
    dst.nbytes = e.nbytes;
    dst.nseg = e.nseg;
    dst.has_split = e.has_split;
    dst.n_empty_rows = e.n_empty_rows;
    prepare_split_combine(L, dst);
    dst.val.ensure((size_t)N + 64);
    if (N > 0)
        SILI_HIP(hipMemcpyAsync(dst.val.p, d_bytes, (size_t)N, hipMemcpyDeviceToDevice, L.stream));
}

void decode_scattered(Layer &L, uint32_t *d_rows, uint32_t *d_cols) {
    const ScaleView none{nullptr, nullptr, 1};
    launch_decode(L.W.plan(), none, reinterpret_cast<int32_t *>(d_cols), nullptr, d_rows, L.stream);
}

void build_shadow(Layer &L, const DScatter &src, const uint32_t *d_rows, const uint32_t *d_cols,
                  DScatter &dst) {
    hipStream_t st = L.stream;
    const int64_t N = src.nnz;
    TmpBuf<uint32_t> keys_out(L, SILI_TMPKEY(keys_out)), perm_in(L, SILI_TMPKEY(perm_in)), perm(L, SILI_TMPKEY(perm)), trows(L, SILI_TMPKEY(trows)), ptrs(L, SILI_TMPKEY(ptrs));
    TmpBuf<uint8_t> tbytes(L, SILI_TMPKEY(tbytes));
    keys_out.ensure((size_t)N + 1);
    perm_in.ensure((size_t)N + 1);
    perm.ensure((size_t)N + 1);
    trows.ensure((size_t)N + 1);
    tbytes.ensure((size_t)N + 1);
    ptrs.ensure((size_t)src.cols + 1);
    // by (column, row): the canonical entries are in (row, column) order, so
    // this is the stable order by column (SILI_SEGSORT=0: a device radix sort)
    zero_flag(L);
    const bool counted = env_int("SILI_SEGSORT", 1) != 0;
    if (counted) sort_major_minor(L, d_cols, d_rows, N, src.cols, perm.p, ptrs.p, L.scratch.flag.p, "shadow build");
    if (!counted && N > 0) {
        launch(k_iota, dim3(nblk(N)), dim3(TPB), 0, st, perm_in.p, N);
        device_sort_pairs_u32(L, d_cols, keys_out.p, perm_in.p, perm.p, N,
                              bits_for((uint64_t)std::max<int64_t>(src.cols - 1, 1)));
    }
    if (N > 0) {
        launch(k_gather_u32, dim3(nblk(N)), dim3(TPB), 0, st, d_rows, perm.p, N, trows.p);
        launch(k_gather_u8, dim3(nblk(N)), dim3(TPB), 0, st, src.val.p, perm.p, N, tbytes.p);
        SILI_HIP(hipGetLastError());
    }
    if (!counted) {
        launch(k_ptrs_from_sorted, dim3(nblk(src.cols + 1)), dim3(TPB), 0, st, keys_out.p, N,
                           src.cols, ptrs.p);
        SILI_HIP(hipGetLastError());
    }
    const Encoded e = encode_rows(L, src.cols, src.rows, N, ptrs.p, trows.p, L.seg_len, true, dst.byte_start,
                                  dst.elem_start, dst.idx, dst.seg, "shadow build", &dst.split_rows);
    dst.n_split = e.n_split;
    dst.stream1.valid = dst.streamK.valid = false;
    dst.stream1.failed = dst.streamK.failed = false;
    dst.fidx.valid = false;
    dst.dcol_valid = false;
    dst.sh_valid = false;
    dst.n_short_hint = e.n_short;
    dst.slc_w = 0;
    dst.cblk.clear();
    dst.cblk_cb = 0;
    dst.rows = src.cols;
    dst.cols = src.rows;
    dst.nnz = N;
    dst.nbytes = e.nbytes;
    dst.nseg = e.nseg;
    dst.has_split = e.has_split;
    dst.n_empty_rows = e.n_empty_rows;
    prepare_split_combine(L, dst);
    dst.val.ensure((size_t)N + 64);
    if (N > 0)
        SILI_HIP(hipMemcpyAsync(dst.val.p, tbytes.p, (size_t)N, hipMemcpyDeviceToDevice, st));
    SILI_HIP(hipStreamSynchronize(st));
    // a training layer keeps the permutation (shadow entry -> canonical
    // entry): its updates rewrite the canonical value bytes and copy them over
    if (&dst == &L.Wt) {
        if (L.keep_perm && N > 0) {
            L.Wt_perm.ensure((size_t)N);
            SILI_HIP(hipMemcpyAsync(L.Wt_perm.p, perm.p, (size_t)N * 4, hipMemcpyDeviceToDevice, st));
            SILI_HIP(hipStreamSynchronize(st));
        } else {
            L.Wt_perm.reset();
        }
    }
}

// Column-block selection: flag entries of block k; gather them with columns
// relative to the block.
__global__ void k_cb_flag(const uint32_t *__restrict__ cols, int64_t N, uint32_t cb, uint32_t k,
                          uint32_t *__restrict__ flag) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i <= N) flag[i] = (i < N && cols[i] / cb == k) ? 1u : 0u;
}
__global__ void k_cb_take(const uint32_t *__restrict__ flag, const uint32_t *__restrict__ pos,
                          const uint32_t *__restrict__ rows, const uint32_t *__restrict__ cols,
                          const uint8_t *__restrict__ val, int64_t N, uint32_t c0, uint32_t *__restrict__ rk,
                          uint32_t *__restrict__ ck, uint8_t *__restrict__ vk) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i >= N || !flag[i]) return;
    const uint32_t j = pos[i];
    rk[j] = rows[i];
    ck[j] = cols[i] - c0;
    vk[j] = val[i];
}

void build_colblocks(Layer &L, DScatter &s, int K, int64_t cb) {
    hipStream_t st = L.stream;
    const int64_t N = s.nnz;
    DevBuf<uint32_t> rows, cols, flag, pos, rk, ck, ptrs;
    DevBuf<uint8_t> vk;
    rows.ensure((size_t)N + 1);
    cols.ensure((size_t)N + 1);
    flag.ensure((size_t)N + 1);
    pos.ensure((size_t)N + 1);
    rk.ensure((size_t)N + 1);
    ck.ensure((size_t)N + 1);
    vk.ensure((size_t)N + 1);
    ptrs.ensure((size_t)s.rows + 1);
    const ScaleView none{nullptr, nullptr, 1};
    if (N > 0) launch_decode(s.plan(), none, reinterpret_cast<int32_t *>(cols.p), nullptr, rows.p, st);
    std::vector<DScatter> blocks((size_t)K);
    for (int k = 0; k < K; ++k) {
        const int64_t c0 = (int64_t)k * cb, ncols = std::min<int64_t>(cb, s.cols - c0);
        launch(k_cb_flag, dim3(nblk(N + 1)), dim3(TPB), 0, st, (const uint32_t *)cols.p, N, (uint32_t)cb,
               (uint32_t)k, flag.p);
        SILI_HIP(hipGetLastError());
        device_exclusive_scan_u32(L, flag.p, pos.p, N + 1);
        uint32_t nk = 0;
        SILI_HIP(hipMemcpyAsync(&nk, pos.p + N, 4, hipMemcpyDeviceToHost, st));
        SILI_HIP(hipStreamSynchronize(st));
        if (N > 0)
            launch(k_cb_take, dim3(nblk(N)), dim3(TPB), 0, st, (const uint32_t *)flag.p, (const uint32_t *)pos.p,
                   (const uint32_t *)rows.p, (const uint32_t *)cols.p, (const uint8_t *)s.val.p, N, (uint32_t)c0,
                   rk.p, ck.p, vk.p);
        launch(k_ptrs_from_sorted, dim3(nblk(s.rows + 1)), dim3(TPB), 0, st, (const uint32_t *)rk.p, (int64_t)nk,
               s.rows, ptrs.p);
        SILI_HIP(hipGetLastError());
        build_scattered(L, blocks[(size_t)k], s.rows, ncols, (int64_t)nk, ptrs.p, ck.p, vk.p);
    }
    s.cblk = std::move(blocks);
    s.cblk_cb = cb;
}

// One orientation of block4 from tiles sorted by (major, minor).
static void build_b4_orientation(Layer &L, DBlock4 &dst, int64_t N, int64_t brows, int64_t bcols,
                                 int64_t rows, int64_t cols, const uint32_t *d_major,
                                 const uint32_t *d_minor, const uint32_t *d_perm,
                                 const uint8_t *d_src_tiles, bool transpose) {
    hipStream_t st = L.stream;
    TmpBuf<uint32_t> ptrs(L, SILI_TMPKEY(ptrs));
    ptrs.ensure((size_t)brows + 1);
    launch(k_ptrs_from_sorted, dim3(nblk(brows + 1)), dim3(TPB), 0, st, d_major, N, brows,
                       ptrs.p);
    SILI_HIP(hipGetLastError());
    const Encoded e = encode_rows(L, brows, bcols, N, ptrs.p, d_minor, L.seg_len_b4, false, dst.byte_start,
                                  dst.tile_start, dst.idx, dst.seg, "block4 build");
    dst.brows = brows;
    dst.bcols = bcols;
    dst.rows = rows;
    dst.cols = cols;
    dst.ntiles = N;
    dst.nbytes = e.nbytes;
    dst.nseg = e.nseg;
    dst.has_split = e.has_split;
    dst.tiles.ensure((size_t)N * 16u + 64);
    dst.cblk.clear();
    dst.cblk_cbb = 0;
    dst.rng_k = 0;
    if (N > 0) {
        launch(k_gather_tiles, dim3(nblk(N)), dim3(TPB), 0, st, d_src_tiles, d_perm, N,
                           transpose ? 1 : 0, dst.tiles.p);
        SILI_HIP(hipGetLastError());
    }
}

// Tiles of block k (minor in [k*cbb, (k+1)*cbb)): major, relative minor and
// storage index, compacted in storage order.
__global__ void k_cb4_take(const uint32_t *__restrict__ flag, const uint32_t *__restrict__ pos,
                           const uint32_t *__restrict__ major, const uint32_t *__restrict__ minor, int64_t N,
                           uint32_t m0, uint32_t *__restrict__ mk, uint32_t *__restrict__ nk,
                           uint32_t *__restrict__ pk) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i >= N || !flag[i]) return;
    const uint32_t j = pos[i];
    mk[j] = major[i];
    nk[j] = minor[i] - m0;
    pk[j] = (uint32_t)i;
}

void build_colblocks_b4(Layer &L, DBlock4 &b, int K, int64_t cbb) {
    hipStream_t st = L.stream;
    const int64_t N = b.ntiles;
    DevBuf<uint32_t> major, minor, flag, pos, mk, nk, pk;
    major.ensure((size_t)N + 1);
    minor.ensure((size_t)N + 1);
    flag.ensure((size_t)N + 1);
    pos.ensure((size_t)N + 1);
    mk.ensure((size_t)N + 1);
    nk.ensure((size_t)N + 1);
    pk.ensure((size_t)N + 1);
    if (N > 0) launch_decode_b4(b.plan(), major.p, minor.p, st);
    std::vector<DBlock4> blocks((size_t)K);
    for (int k = 0; k < K; ++k) {
        const int64_t m0 = (int64_t)k * cbb;
        const int64_t nbc = std::min<int64_t>(cbb, b.bcols - m0);
        const int64_t c0 = m0 * 4, ncols = std::min<int64_t>(nbc * 4, b.cols - c0);
        launch(k_cb_flag, dim3(nblk(N + 1)), dim3(TPB), 0, st, (const uint32_t *)minor.p, N, (uint32_t)cbb,
               (uint32_t)k, flag.p);
        SILI_HIP(hipGetLastError());
        device_exclusive_scan_u32(L, flag.p, pos.p, N + 1);
        uint32_t nt = 0;
        SILI_HIP(hipMemcpyAsync(&nt, pos.p + N, 4, hipMemcpyDeviceToHost, st));
        SILI_HIP(hipStreamSynchronize(st));
        if (N > 0)
            launch(k_cb4_take, dim3(nblk(N)), dim3(TPB), 0, st, (const uint32_t *)flag.p, (const uint32_t *)pos.p,
                   (const uint32_t *)major.p, (const uint32_t *)minor.p, N, (uint32_t)m0, mk.p, nk.p, pk.p);
        SILI_HIP(hipGetLastError());
        build_b4_orientation(L, blocks[(size_t)k], (int64_t)nt, b.brows, nbc, b.rows, ncols, mk.p, nk.p, pk.p,
                             b.tiles.p, false);
    }
    SILI_HIP(hipStreamSynchronize(st));
    b.cblk = std::move(blocks);
    b.cblk_cbb = cbb;
}

// start[x*brows + br] = the first tile of block row br whose block column
// is >= x * cbb (x < K), start[K*brows + br] = the row's end.
__global__ void k_range_starts(const uint32_t *__restrict__ tile_start, const uint32_t *__restrict__ tcol,
                               int64_t brows, int64_t K, int64_t cbb, uint32_t *__restrict__ start) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i >= (K + 1) * brows) return;
    const int64_t x = i / brows, br = i % brows;
    uint32_t lo = tile_start[br], hi = tile_start[br + 1];
    if (x == K) {
        start[i] = hi;
        return;
    }
    const uint64_t key = (uint64_t)x * (uint64_t)cbb;
    while (lo < hi) {
        const uint32_t mid = lo + ((hi - lo) >> 1);
        if ((uint64_t)tcol[mid] < key) lo = mid + 1;
        else hi = mid;
    }
    start[i] = lo;
}

void ensure_col_ranges(Layer &L, DBlock4 &b, int K) {
    if (K < 1) throw_error(1, "column ranges: K must be >= 1");
    if (b.rng_k == K) return;
    hipStream_t st = L.stream;
    const int64_t N = b.ntiles;
    b.rng_col.ensure((size_t)N + 1);
    b.rng_start.ensure((size_t)(K + 1) * (size_t)b.brows + 1);
    DevBuf<uint32_t> major;
    major.ensure((size_t)N + 1);
    if (N > 0) launch_decode_b4(b.plan(), major.p, b.rng_col.p, st);
    const int64_t cbb = (b.bcols + K - 1) / K;
    const int64_t n = (int64_t)(K + 1) * b.brows;
    if (n > 0)
        launch(k_range_starts, dim3(nblk(n)), dim3(TPB), 0, st, (const uint32_t *)b.tile_start.p,
               (const uint32_t *)b.rng_col.p, b.brows, (int64_t)K, cbb, b.rng_start.p);
    SILI_HIP(hipGetLastError());
    SILI_HIP(hipStreamSynchronize(st));
    b.rng_k = K;
}

void build_block4(Layer &L, int64_t n_tiles, const uint32_t *d_br, const uint32_t *d_bc,
                  const uint8_t *d_tiles, const uint8_t *d_flags, int64_t sorted_head) {
    hipStream_t st = L.stream;
    const int64_t brows = (L.n_in + 3) / 4, bcols = (L.n_out + 3) / 4;
    const int64_t N = n_tiles;
    TmpBuf<uint64_t> key(L, SILI_TMPKEY(key)), key_sorted(L, SILI_TMPKEY(key_sorted));
    TmpBuf<uint32_t> perm_in(L, SILI_TMPKEY(perm_in)), perm(L, SILI_TMPKEY(perm)), major(L, SILI_TMPKEY(major)), minor(L, SILI_TMPKEY(minor));
    TmpBuf<uint32_t> inv(L, SILI_TMPKEY(inv)), mptr(L, SILI_TMPKEY(mptr));
    key.ensure((size_t)N + 1);
    key_sorted.ensure((size_t)N + 1);
    perm_in.ensure((size_t)N + 1);
    perm.ensure((size_t)N + 1);
    major.ensure((size_t)N + 1);
    minor.ensure((size_t)N + 1);
    for (int orient = 0; orient < 2; ++orient) {
        const bool canon = orient == 0;
        const uint32_t *maj = canon ? d_br : d_bc;
        const uint32_t *mnr = canon ? d_bc : d_br;
        const int64_t maj_ext = canon ? brows : bcols, mnr_ext = canon ? bcols : brows;
        zero_flag(L);
        if (N > 0) {
            launch(k_tile_keys, dim3(nblk(N)), dim3(TPB), 0, st, maj, mnr, N,
                               (uint64_t)mnr_ext, maj_ext, key.p, L.scratch.flag.p);
            launch(k_iota, dim3(nblk(N)), dim3(TPB), 0, st, perm_in.p, N);
            SILI_HIP(hipGetLastError());
            if (canon && sorted_head >= 0 && sorted_head <= N) {
                // two runs already in canonical order: merged, not sorted
                // (k_split_keys flags a merge whose runs were not)
                device_merge_pairs_u64(L, key.p, key.p + sorted_head, key_sorted.p, perm_in.p,
                                       perm_in.p + sorted_head, perm.p, sorted_head, N - sorted_head);
            } else if (env_int("SILI_SEGSORT", 1)) {
                // counted by major, each major's tiles ordered by minor
                mptr.ensure((size_t)maj_ext + 1);
                sort_major_minor(L, maj, mnr, N, maj_ext, perm.p, mptr.p, L.scratch.flag.p, "block4 tiles");
                launch(k_gather_u64, dim3(nblk(N)), dim3(TPB), 0, st, (const uint64_t *)key.p, (const uint32_t *)perm.p,
                       N, key_sorted.p);
            } else {
                device_sort_pairs_u64(L, key.p, key_sorted.p, perm_in.p, perm.p, N,
                                      bits_for((uint64_t)maj_ext * (uint64_t)mnr_ext));
            }
            launch(k_split_keys, dim3(nblk(N)), dim3(TPB), 0, st, key_sorted.p, N,
                               (uint64_t)mnr_ext, major.p, minor.p, L.scratch.flag.p);
            SILI_HIP(hipGetLastError());
        }
        // (a build from the layer's own arrays: its tiles are in range and
        // its merged runs were checked in order before)
        if (!L.trusted_build) check_flag(L, L.scratch.flag.p, "block4 tiles");
        if (canon) {
            build_b4_orientation(L, L.B4, N, brows, bcols, L.n_in, L.n_out, major.p, minor.p, perm.p,
                                 d_tiles, false);
            inv.ensure((size_t)N + 1);
            if (N > 0) launch(k_inv_perm, dim3(nblk(N)), dim3(TPB), 0, st, (const uint32_t *)perm.p, N, inv.p);
            // tile_is_sparse of the canonical tiles: carried through the sort,
            // or (a load) every tile encoded by its live count
            L.B4.sparse.ensure((size_t)N + 1);
            if (N > 0 && d_flags)
                launch(k_gather_u8, dim3(nblk(N)), dim3(TPB), 0, st, d_flags, (const uint32_t *)perm.p, N,
                       L.B4.sparse.p);
            else if (N > 0)
                tiles_reencode(L, nullptr, st);
        } else {
            build_b4_orientation(L, L.B4t, N, bcols, brows, L.n_out, L.n_in, major.p, minor.p, perm.p,
                                 d_tiles, true);
            // shadow tile -> canonical tile (the update refreshes the shadow through it)
            L.B4t_perm.ensure((size_t)N + 1);
            if (N > 0)
                launch(k_compose_perm, dim3(nblk(N)), dim3(TPB), 0, st, (const uint32_t *)perm.p,
                       (const uint32_t *)inv.p, N, L.B4t_perm.p);
        }
        SILI_HIP(hipGetLastError());
    }
    SILI_HIP(hipStreamSynchronize(st));
}

void launch_b4_shadow_refresh(Layer &L, hipStream_t st) {
    if (L.B4.ntiles == 0) return;
    ProfScope ps("train_b4_shadow", st);
    launch(k_gather_tiles, dim3(nblk(L.B4.ntiles)), dim3(TPB), 0, st, (const uint8_t *)L.B4.tiles.p,
           (const uint32_t *)L.B4t_perm.p, L.B4.ntiles, 1, L.B4t.tiles.p);
    SILI_HIP(hipGetLastError());
}

void refresh_nonfinite(Layer &L) {
    hipStream_t st = L.stream;
    zero_flag(L);
    if (L.W.nnz > 0)
        launch(k_scan_nan_codes, dim3(nblk(L.W.nnz)), dim3(TPB), 0, st, L.W.val.p, L.W.nnz, 1,
                           L.scratch.flag.p);
    if (L.B4.ntiles > 0)
        launch(k_scan_nan_codes, dim3(nblk(L.B4.ntiles * 16)), dim3(TPB), 0, st, L.B4.tiles.p,
                           L.B4.ntiles * 16, 0, L.scratch.flag.p);
    SILI_HIP(hipGetLastError());
    int h = 0;
    SILI_HIP(hipMemcpyAsync(&h, L.scratch.flag.p, sizeof(int), hipMemcpyDeviceToHost, st));
    SILI_HIP(hipStreamSynchronize(st));
    L.has_nonfinite = (h != 0) || L.nonfinite_scales;
}

}  // namespace sili
