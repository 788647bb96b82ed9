// gen.hip -- seeded synthetic layers generated on the device (benchmark
// workloads too large to build on the host, e.g. the folded-transformer
// shapes with billions of synapses).
//
// Synapse (r, c) exists iff the high word of h = mix64(seed, r, c) is below
// keep_prob * 2^32 (an integer decision, identical on any host).  Its weight
// magnitude is sigma * sqrt(2) * erfinv(a + (1 - a) * u) with
// a = 2 * tail_q - 1 and u in (0, 1) from 24 bits of h (computed through
// erfcinv of the complement, finite for every u): the |N(0, sigma)|
// distribution conditioned on |w| >= sigma * Phi^-1(tail_q) (tail_q = 0.5:
// plain half-normal); bit 0 of h is the sign.  Quantisation follows the
// reference's per-row recipe (sili/sparse_rnn.py:1022-1037):
// s_r = fl32(fl64(max_row |w|) / 6), code = fp4_encode(fl32(w / s_r)),
// importance 0.  The rows are then encoded by the same device builders as
// any load (delta-CSR + shadow).
#include "layer.hpp"
#include "wave.hpp"

namespace sili {

namespace {

constexpr unsigned TPB = 256;

// 64-bit finaliser (MurmurHash3 fmix64; public domain) over a mixed key.
__device__ __forceinline__ uint64_t fmix64(uint64_t k) {
    k ^= k >> 33;
    k *= 0xff51afd7ed558ccdull;
    k ^= k >> 33;
    k *= 0xc4ceb9fe1a85ec53ull;
    k ^= k >> 33;
    return k;
}
__device__ __forceinline__ uint64_t syn_hash(uint64_t seed, uint32_t r, uint32_t c) {
    return fmix64(seed ^ ((uint64_t)r * 0x9E3779B97F4A7C15ull) ^ ((uint64_t)c * 0xD1B54A32D192ED03ull));
}
// erfinv(a + (1 - a) u) evaluated as erfcinv((1 - a)(1 - u)): the argument
// stays > 0 for every 24-bit u (a + (1 - a) u itself can round to 1.0f, where
// erfinv is infinite).
__device__ __forceinline__ float syn_weight(uint64_t h, float sigma, float a) {
    const float one_minus_u = ((float)(16777215u - (uint32_t)((h >> 8) & 0xFFFFFFu)) + 0.5f) * (1.0f / 16777216.0f);
    const float m = sigma * 1.41421356237f * erfcinvf((1.0f - a) * one_minus_u);
    return (h & 1u) ? -m : m;
}

struct GenArgs {
    uint64_t seed;
    uint32_t thr;  // keep iff (h >> 32) < thr
    float sigma, a;
    int64_t n_in, n_out;
};

// Pass A: one wave per row -- kept count and max |w|.
__global__ __launch_bounds__(256) void k_gen_count(GenArgs g, uint32_t *count, float *rmax) {
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= g.n_in) return;
    const uint32_t lane = threadIdx.x & 63u;
    uint32_t n = 0;
    float mx = 0.0f;
    for (int64_t c0 = 0; c0 < g.n_out; c0 += 64) {
        const int64_t c = c0 + lane;
        if (c < g.n_out) {
            const uint64_t h = syn_hash(g.seed, (uint32_t)r, (uint32_t)c);
            if ((uint32_t)(h >> 32) < g.thr) {
                ++n;
                mx = fmaxf(mx, __builtin_fabsf(syn_weight(h, g.sigma, g.a)));
            }
        }
    }
    // wave reductions (sum, max) through the DPP scan helpers
    const uint32_t tot = uniform(__builtin_amdgcn_readlane((int)wave_incl_scan(n), 63));
    for (uint32_t off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, (int)off, 64));
    if (lane == 0) {
        count[r] = tot;
        rmax[r] = mx;
    }
}

// Pass B: one wave per row -- columns (ascending), value bytes, row ids.
__global__ __launch_bounds__(256) void k_gen_write(GenArgs g, const uint32_t *ptrs, const float *scale,
                                                   uint32_t *cols, uint8_t *bytes, uint32_t *rows) {
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= g.n_in) return;
    const uint32_t lane = threadIdx.x & 63u;
    const float s = scale[r];
    uint32_t base = ptrs[r];
    for (int64_t c0 = 0; c0 < g.n_out; c0 += 64) {
        const int64_t c = c0 + lane;
        bool keep = false;
        uint64_t h = 0;
        if (c < g.n_out) {
            h = syn_hash(g.seed, (uint32_t)r, (uint32_t)c);
            keep = (uint32_t)(h >> 32) < g.thr;
        }
        const uint64_t K = __ballot(keep);
        if (keep) {
            const uint32_t rank = __builtin_amdgcn_mbcnt_hi((uint32_t)(K >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)K, 0u));
            const float w = syn_weight(h, g.sigma, g.a);
            const uint32_t code = fp4_encode(w / s);
            cols[base + rank] = (uint32_t)c;
            bytes[base + rank] = (uint8_t)(code << 4);
            rows[base + rank] = (uint32_t)r;
        }
        base += (uint32_t)__popcll(K);
    }
}

// s_r = fl32(fl64(max) / 6); rows without synapses keep scale 1.
__global__ void k_gen_scale(const float *rmax, int64_t n, float *scale) {
    const int64_t r = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (r >= n) return;
    const float m = rmax[r];
    scale[r] = m > 0.0f ? (float)((double)m / 6.0) : 1.0f;
}

}  // namespace

int64_t generate_synthetic(Layer &L, uint64_t seed, double keep_prob, float sigma, float tail_q) {
    hipStream_t st = L.stream;
    const int64_t n_in = L.n_in, n_out = L.n_out;
    GenArgs g{seed, (uint32_t)std::min(4294967295.0, keep_prob * 4294967296.0), sigma, 2.0f * tail_q - 1.0f,
              n_in, n_out};
    DevBuf<uint32_t> count, ptrs;
    DevBuf<float> rmax;
    count.ensure((size_t)n_in + 1);
    ptrs.ensure((size_t)n_in + 1);
    rmax.ensure((size_t)n_in);
    const unsigned rows_blocks = (unsigned)((n_in + 3) / 4);
    launch(k_gen_count, dim3(rows_blocks), dim3(256), 0, st, g, count.p, rmax.p);
    launch(k_gen_scale, dim3((unsigned)((n_in + TPB - 1) / TPB)), dim3(TPB), 0, st, (const float *)rmax.p, n_in,
           L.vs.p);
    SILI_HIP(hipGetLastError());
    // ptrs = exclusive scan of the counts (count[n_in] = 0 gives the total)
    const uint32_t zero = 0;
    SILI_HIP(hipMemcpyAsync(count.p + n_in, &zero, 4, hipMemcpyHostToDevice, st));
    device_exclusive_scan_u32(L, count.p, ptrs.p, n_in + 1);
    uint32_t nnz32 = 0;
    SILI_HIP(hipMemcpyAsync(&nnz32, ptrs.p + n_in, 4, hipMemcpyDeviceToHost, st));
    SILI_HIP(hipStreamSynchronize(st));
    const int64_t nnz = nnz32;
    if (nnz >= (int64_t(1) << 31) - 1) throw_error(4, "synthetic layer: more than 2^31 synapses");
    DevBuf<uint32_t> cols, rows;
    DevBuf<uint8_t> bytes;
    cols.ensure((size_t)nnz + 1);
    rows.ensure((size_t)nnz + 1);
    bytes.ensure((size_t)nnz + 1);
    launch(k_gen_write, dim3(rows_blocks), dim3(256), 0, st, g, (const uint32_t *)ptrs.p, (const float *)L.vs.p,
           cols.p, bytes.p, rows.p);
    SILI_HIP(hipGetLastError());
    L.idx_budget = std::max<int64_t>(L.idx_budget, nnz * 8 + 4096);
    L.val_budget = std::max<int64_t>(L.val_budget, nnz + 64);
    build_scattered(L, L.W, n_in, n_out, nnz, ptrs.p, cols.p, bytes.p);
    build_shadow(L, L.W, rows.p, cols.p, L.Wt);
    return nnz;
}

}  // namespace sili
