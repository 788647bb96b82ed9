// probes.hip -- measurement probes behind the kernels' design choices (not
// part of the layer library; bench.py --probe runs them):
//
//   load: random 256-byte row loads from a small table through the per-CU
//         load path, in the gathers' lane layouts (BL lanes per row, float4
//         chunks, U rows in flight per lane) -- the ceiling the segment
//         gathers are measured against;
//   lds:  LDS read throughput (bytes per clock per CU) of the access
//         patterns the staged-input gather chose between.
//
// Every access is in bounds (indices are masked to the table) and every
// wave runs a fixed number of iterations.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <vector>

namespace {

// Random rows: entry e reads row idx[e] (64 fp32 = 256 bytes) of `table`;
// BL lanes per row, each owning 64 / (4 BL) float4 chunks; G = 64 / BL rows
// per load instruction, U instructions in flight.
template <int BL, int U>
__global__ __launch_bounds__(256) void k_probe_rows(const float4 *__restrict__ table, const uint32_t *__restrict__ idx,
                                                    int64_t n, float *__restrict__ out) {
    constexpr int KB = 16 / BL;  // float4 chunks per lane (a row is 16 float4)
    constexpr int G = 64 / BL;
    const uint32_t lane = threadIdx.x & 63u, g = lane / BL, bl = lane % BL;
    const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int64_t nwaves = ((int64_t)gridDim.x * blockDim.x) >> 6;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int64_t base = wave * G * U; base < n; base += nwaves * G * U) {
        float4 x[U][KB];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t e = base + u * G + g;
            const uint32_t r = e < n ? idx[e] : 0u;
#pragma unroll
            for (int k = 0; k < KB; ++k) x[u][k] = table[(size_t)r * 16u + bl + BL * k];
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int k = 0; k < KB; ++k) {
                acc.x += x[u][k].x;
                acc.y += x[u][k].y;
                acc.z += x[u][k].z;
                acc.w += x[u][k].w;
            }
    }
    out[(int64_t)blockIdx.x * blockDim.x + threadIdx.x] = acc.x + acc.y + acc.z + acc.w;
}

// LDS patterns over 257 rows of `stride` floats; each lane reads 32 bytes
// per iteration (two float4), one random row per group of 16 lanes:
//   0: two chunks per lane at 4 sub and 64 + 4 sub, rows 512 bytes apart;
//   1: the same with a 16-byte skew between rows (stride 132 floats);
//   2: 32-lane halves, one row each, 16 bytes per lane, two rows per step.
constexpr int LDS_ITERS = 2048;
template <int MODE>
__global__ __launch_bounds__(1024) void k_probe_lds(float *__restrict__ out, uint32_t seed) {
    extern __shared__ __align__(16) float xs[];
    constexpr uint32_t STRIDE = MODE == 1 ? 132u : 128u;
    const uint32_t t = threadIdx.x, lane = t & 63u, sub = lane & 15u;
    for (uint32_t i = t; i < 257u * STRIDE; i += 1024u) xs[i] = (float)(i & 7u);
    __syncthreads();
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    uint32_t r = seed * 747796405u + t * 2891336453u;
    for (int it = 0; it < LDS_ITERS; ++it) {
        r = r * 1664525u + 1013904223u;
        const uint32_t rowg = (uint32_t)__shfl((int)(r >> 8), (int)(lane & ~15u), 64) & 255u;
        const uint32_t row32 = (uint32_t)__shfl((int)(r >> 8), (int)(lane & ~31u), 64) & 255u;
        float4 a, b;
        if (MODE == 2) {
            const uint32_t l32 = lane & 31u;
            a = *(const float4 *)(xs + row32 * STRIDE + l32 * 4u);
            b = *(const float4 *)(xs + ((row32 + 7u) & 255u) * STRIDE + l32 * 4u);
        } else {
            const float *p = xs + rowg * STRIDE + sub * 4u;
            a = *(const float4 *)p;
            b = *(const float4 *)(p + 64);
        }
        acc.x += a.x + b.x;
        acc.y += a.y + b.y;
        acc.z += a.z + b.z;
        acc.w += a.w + b.w;
    }
    if (acc.x == 12345.0f) out[t] = acc.y + acc.z + acc.w;  // never true: keeps the reads
}

int run_ms(hipEvent_t e0, hipEvent_t e1, double *ms) {
    float f = 0;
    if (hipEventSynchronize(e1) != hipSuccess || hipEventElapsedTime(&f, e0, e1) != hipSuccess) return 1;
    *ms = f;
    return 0;
}

}  // namespace

extern "C" {

// Random-row load probe: n_entries rows drawn (seeded) from a table of
// n_rows rows of 256 bytes, BL lanes per row (4, 8 or 16), U = 4 in flight;
// best of `reps` launches.  Returns 0 and the milliseconds, else non-zero.
int sili_probe_load_rows(int bl, int64_t n_rows, int64_t n_entries, int reps, double *ms_out) {
    if (!ms_out || n_rows <= 0 || n_entries <= 0 || reps <= 0 || (bl != 4 && bl != 8 && bl != 16)) return 1;
    std::vector<uint32_t> h((size_t)n_entries);
    uint64_t s = 0x9E3779B97F4A7C15ull;
    for (auto &v : h) {
        s ^= s << 13;
        s ^= s >> 7;
        s ^= s << 17;
        v = (uint32_t)(s % (uint64_t)n_rows);
    }
    float4 *table = nullptr;
    uint32_t *idx = nullptr;
    float *out = nullptr;
    const unsigned blocks = 2048, threads = 256;
    if (hipMalloc(&table, (size_t)n_rows * 256) != hipSuccess) return 2;
    if (hipMalloc(&idx, (size_t)n_entries * 4) != hipSuccess) return 2;
    if (hipMalloc(&out, (size_t)blocks * threads * 4) != hipSuccess) return 2;
    if (hipMemset(table, 0, (size_t)n_rows * 256) != hipSuccess) return 3;
    if (hipMemcpy(idx, h.data(), (size_t)n_entries * 4, hipMemcpyHostToDevice) != hipSuccess) return 3;
    hipEvent_t e0, e1;
    if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) return 4;
    double best = 1e30;
    for (int rep = 0; rep <= reps; ++rep) {  // rep 0 warms up
        hipEventRecord(e0);
        if (bl == 4) k_probe_rows<4, 4><<<blocks, threads>>>(table, idx, n_entries, out);
        else if (bl == 8) k_probe_rows<8, 4><<<blocks, threads>>>(table, idx, n_entries, out);
        else k_probe_rows<16, 4><<<blocks, threads>>>(table, idx, n_entries, out);
        hipEventRecord(e1);
        double ms = 0;
        if (hipGetLastError() != hipSuccess || run_ms(e0, e1, &ms)) return 5;
        if (rep > 0 && ms < best) best = ms;
    }
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    hipFree(table);
    hipFree(idx);
    hipFree(out);
    *ms_out = best;
    return 0;
}

// LDS pattern probe (mode 0, 1 or 2 above): LDS bytes read per clock per CU,
// one block of 1024 threads per CU slot, 4 blocks per CU, best of `reps`.
int sili_probe_lds(int mode, int reps, double *bytes_per_clk_cu) {
    if (!bytes_per_clk_cu || reps <= 0 || mode < 0 || mode > 2) return 1;
    int dev = 0, clk_khz = 0, ncu = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 2;
    hipDeviceGetAttribute(&clk_khz, hipDeviceAttributeClockRate, dev);
    hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev);
    if (clk_khz <= 0 || ncu <= 0) return 2;
    const int lds = 257 * 132 * 4;
    const void *f = mode == 0 ? (const void *)k_probe_lds<0> : mode == 1 ? (const void *)k_probe_lds<1>
                                                                         : (const void *)k_probe_lds<2>;
    if (hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, lds) != hipSuccess) return 3;
    float *out = nullptr;
    if (hipMalloc(&out, 1024 * 4) != hipSuccess) return 3;
    hipEvent_t e0, e1;
    if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) return 4;
    const int grid = ncu * 4;
    double best = 1e30;
    for (int rep = 0; rep <= reps; ++rep) {
        hipEventRecord(e0);
        if (mode == 0) k_probe_lds<0><<<grid, 1024, lds>>>(out, (uint32_t)rep + 1u);
        else if (mode == 1) k_probe_lds<1><<<grid, 1024, lds>>>(out, (uint32_t)rep + 1u);
        else k_probe_lds<2><<<grid, 1024, lds>>>(out, (uint32_t)rep + 1u);
        hipEventRecord(e1);
        double ms = 0;
        if (hipGetLastError() != hipSuccess || run_ms(e0, e1, &ms)) return 5;
        if (rep > 0 && ms < best) best = ms;
    }
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    hipFree(out);
    const double bytes = (double)grid * 1024.0 * LDS_ITERS * 32.0;
    *bytes_per_clk_cu = bytes / ncu / (best * 1e-3 * (double)clk_khz * 1e3);
    return 0;
}

}  // extern "C"
