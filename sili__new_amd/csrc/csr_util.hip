// csr_util.hip -- the module's CSR construction utilities on the device:
// dense_to_csr (threshold) and dense_to_top_k_csr (global top-k by
// magnitude), the two conversions the reference's layers apply to
// activations and gradients before the sparse-input paths
// (sili/cpu_backend.cpp:3075-3156; SISLDOLayer.backward calls the top-k one,
// sili/sparse_rnn.py:802).
//
// Inputs and outputs are device buffers; each call runs on the given stream
// and synchronizes it once, to report the entry count to the host.
#include "../../include/sili_hip.h"
#include "layer.hpp"
#include "wave.hpp"

#include <algorithm>
#include <vector>
#include <cstring>  // host memset, needed before rocprim's headers

#include <rocprim/rocprim.hpp>

namespace sili {

namespace {

constexpr unsigned TPB = 256;
inline unsigned nblk(int64_t n) { return (unsigned)((n + TPB - 1) / TPB); }

// The reference's keep rule: v > t || v < -t (so NaN is never kept).
__device__ __forceinline__ bool keep(float v, float t) { return v > t || v < -t; }

// counts[r] = entries of row r kept (one block per row).
__global__ __launch_bounds__(TPB) void k_row_keep_count(const float *__restrict__ x, int64_t cols, float t,
                                                        uint32_t *__restrict__ counts) {
    __shared__ uint32_t s_part[TPB / 64];
    const int64_t r = blockIdx.x;
    const float *row = x + r * cols;
    uint32_t n = 0;
    for (int64_t c = threadIdx.x; c < cols; c += TPB) n += keep(row[c], t) ? 1u : 0u;
    // wave sum, then the block's waves
    uint32_t s = n;
    for (int off = 32; off > 0; off >>= 1) s += (uint32_t)__shfl_xor((int)s, off, 64);
    if ((threadIdx.x & 63u) == 0u) s_part[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t tot = 0;
        for (unsigned w = 0; w < TPB / 64; ++w) tot += s_part[w];
        counts[r] = tot;
    }
}

// Row r's kept entries, in column order, at ptrs[r] (one block per row:
// 256-column chunks, ballots give each kept entry its rank in the chunk).
__global__ __launch_bounds__(TPB) void k_row_keep_fill(const float *__restrict__ x, int64_t cols, float t,
                                                       const uint32_t *__restrict__ ptrs,
                                                       int32_t *__restrict__ idx, float *__restrict__ vals) {
    __shared__ uint32_t s_cnt[TPB / 64];
    const int64_t r = blockIdx.x;
    const float *row = x + r * cols;
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    uint32_t base = ptrs[r];
    for (int64_t c0 = 0; c0 < cols; c0 += TPB) {
        const int64_t c = c0 + threadIdx.x;
        const float v = c < cols ? row[c] : 0.0f;
        const bool k = c < cols && keep(v, t);
        const uint64_t m = __ballot(k);
        const uint32_t rank = __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
        if (lane == 0u) s_cnt[wave] = (uint32_t)__popcll(m);
        __syncthreads();
        uint32_t before = 0, total = 0;
        for (uint32_t w = 0; w < TPB / 64; ++w) {
            before += w < wave ? s_cnt[w] : 0u;
            total += s_cnt[w];
        }
        if (k) {
            idx[base + before + rank] = (int32_t)c;
            vals[base + before + rank] = v;
        }
        base += total;
        __syncthreads();  // s_cnt is rewritten by the next chunk
    }
}

// key = magnitude bits (sign cleared; monotone in |v| for non-NaN floats),
// value = flat index.
__global__ void k_mag_keys(const float *__restrict__ x, int64_t n, uint32_t *__restrict__ key,
                           uint32_t *__restrict__ flat) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i >= n) return;
    key[i] = __builtin_bit_cast(uint32_t, x[i]) & 0x7FFFFFFFu;
    flat[i] = (uint32_t)i;
}

// COO (flat indices ascending) -> CSR columns and values; ptrs[r] = first
// entry with flat index >= r * cols (binary search).
__global__ void k_topk_entries(const uint32_t *__restrict__ flat, int64_t k, int64_t cols,
                               const float *__restrict__ x, int32_t *__restrict__ idx, float *__restrict__ vals) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i >= k) return;
    const uint32_t f = flat[i];
    idx[i] = (int32_t)((int64_t)f % cols);
    vals[i] = x[f];
}
__global__ void k_topk_ptrs(const uint32_t *__restrict__ flat, int64_t k, int64_t rows, int64_t cols,
                            int32_t *__restrict__ ptrs) {
    const int64_t r = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (r > rows) return;
    const uint64_t lim = (uint64_t)r * (uint64_t)cols;
    int64_t lo = 0, hi = k;
    while (lo < hi) {
        const int64_t mid = (lo + hi) >> 1;
        if ((uint64_t)flat[mid] < lim) lo = mid + 1;
        else hi = mid;
    }
    ptrs[r] = (int32_t)lo;
}

__global__ void k_u32_to_i32(const uint32_t *__restrict__ s, int64_t n, int32_t *__restrict__ d) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i < n) d[i] = (int32_t)s[i];
}

}  // namespace

void dense_to_csr_device(const float *x, int64_t rows, int64_t cols, float threshold, int32_t *ptrs, int32_t *idx,
                         float *vals, int64_t cap, int64_t *nnz, hipStream_t st) {
    if (rows < 0 || cols < 0) throw_error(SILI_ERR_INVALID, "dense_to_csr: negative shape");
    if (rows * cols >= (int64_t(1) << 31)) throw_error(SILI_ERR_INVALID, "dense_to_csr: more than 2^31 - 1 elements");
    if (!ptrs || (rows > 0 && cols > 0 && !x)) throw_error(SILI_ERR_INVALID, "dense_to_csr: NULL buffer");
    DevBuf<uint32_t> cnt, off;
    DevBuf<uint8_t> temp;
    cnt.ensure((size_t)rows + 1);
    off.ensure((size_t)rows + 1);
    SILI_HIP(hipMemsetAsync(cnt.p, 0, ((size_t)rows + 1) * sizeof(uint32_t), st));
    if (rows > 0 && cols > 0) launch(k_row_keep_count, dim3((unsigned)rows), dim3(TPB), 0, st, x, cols, threshold, cnt.p);
    size_t bytes = 0;
    SILI_HIP(rocprim::exclusive_scan(nullptr, bytes, cnt.p, off.p, uint32_t(0), (size_t)rows + 1,
                                     rocprim::plus<uint32_t>(), st));
    temp.ensure(bytes + 16);
    SILI_HIP(rocprim::exclusive_scan(temp.p, bytes, cnt.p, off.p, uint32_t(0), (size_t)rows + 1,
                                     rocprim::plus<uint32_t>(), st));
    uint32_t total = 0;
    SILI_HIP(hipMemcpyAsync(&total, off.p + rows, sizeof(uint32_t), hipMemcpyDeviceToHost, st));
    launch(k_u32_to_i32, dim3(nblk(rows + 1)), dim3(TPB), 0, st, (const uint32_t *)off.p, rows + 1, ptrs);
    SILI_HIP(hipStreamSynchronize(st));
    *nnz = (int64_t)total;
    if ((int64_t)total > cap)
        throw_error(SILI_ERR_RANGE, "dense_to_csr: " + std::to_string(total) + " entries exceed the capacity of " +
                                        std::to_string(cap));
    if (total > 0) {
        if (!idx || !vals) throw_error(SILI_ERR_INVALID, "dense_to_csr: NULL output buffer");
        launch(k_row_keep_fill, dim3((unsigned)rows), dim3(TPB), 0, st, x, cols, threshold,
               (const uint32_t *)off.p, idx, vals);
    }
    SILI_HIP(hipGetLastError());
    SILI_HIP(hipStreamSynchronize(st));
}

void dense_to_top_k_csr_device(const float *x, int64_t rows, int64_t cols, int64_t k, int32_t *ptrs, int32_t *idx,
                               float *vals, int64_t *nnz, hipStream_t st) {
    if (rows < 0 || cols < 0 || k < 0) throw_error(SILI_ERR_INVALID, "dense_to_top_k_csr: negative argument");
    const int64_t n = rows * cols;
    if (n >= (int64_t(1) << 31)) throw_error(SILI_ERR_INVALID, "dense_to_top_k_csr: more than 2^31 - 1 elements");
    if (!ptrs || (n > 0 && !x)) throw_error(SILI_ERR_INVALID, "dense_to_top_k_csr: NULL buffer");
    const int64_t kk = std::min(k, n);  // top_k_indices clamps k to the size (csr.hpp:413)
    *nnz = kk;
    if (kk == 0) {
        std::vector<int32_t> h((size_t)rows + 1, 0);
        SILI_HIP(hipMemcpyAsync(ptrs, h.data(), h.size() * sizeof(int32_t), hipMemcpyHostToDevice, st));
        SILI_HIP(hipStreamSynchronize(st));
        return;
    }
    if (!idx || !vals) throw_error(SILI_ERR_INVALID, "dense_to_top_k_csr: NULL output buffer");
    DevBuf<uint32_t> key, key2, flat, flat2, sel, sel2;
    DevBuf<uint8_t> temp;
    key.ensure((size_t)n);
    key2.ensure((size_t)n);
    flat.ensure((size_t)n);
    flat2.ensure((size_t)n);
    launch(k_mag_keys, dim3(nblk(n)), dim3(TPB), 0, st, x, n, key.p, flat.p);
    // descending magnitude; the radix sort is stable, so equal magnitudes
    // keep ascending flat order (the lowest flat index wins a tie at the cut)
    size_t bytes = 0;
    SILI_HIP(rocprim::radix_sort_pairs_desc(nullptr, bytes, key.p, key2.p, flat.p, flat2.p, (size_t)n, 0u, 32u, st));
    temp.ensure(bytes + 16);
    SILI_HIP(rocprim::radix_sort_pairs_desc(temp.p, bytes, key.p, key2.p, flat.p, flat2.p, (size_t)n, 0u, 32u, st));
    // the kept flat indices in row-major order (merge_sort_coo, csr.hpp:499)
    sel.ensure((size_t)kk);
    size_t bytes2 = 0;
    SILI_HIP(rocprim::radix_sort_keys(nullptr, bytes2, flat2.p, sel.p, (size_t)kk, 0u, 32u, st));
    if (bytes2 + 16 > temp.n) temp.ensure(bytes2 + 16);
    SILI_HIP(rocprim::radix_sort_keys(temp.p, bytes2, flat2.p, sel.p, (size_t)kk, 0u, 32u, st));
    launch(k_topk_entries, dim3(nblk(kk)), dim3(TPB), 0, st, (const uint32_t *)sel.p, kk, cols, x, idx, vals);
    launch(k_topk_ptrs, dim3(nblk(rows + 1)), dim3(TPB), 0, st, (const uint32_t *)sel.p, kk, rows, cols, ptrs);
    SILI_HIP(hipGetLastError());
    SILI_HIP(hipStreamSynchronize(st));
}

}  // namespace sili
