// staged.hip -- the dense-input forward at batches 65..128 with the input
// staged in LDS (linear_disldo.hpp:68-126: y[b, j] = sum_i x[b, i] W[i, j],
// here over the shadow store, rows = outputs j).
//
// The segment gather loads a synapse's whole input row (B fp32 values) from
// L2 for every synapse: at batch 128 that is 512 bytes per synapse through
// the per-CU load path, which bounds it.  Here a block of 1024 threads owns
// 128 consecutive output rows and sweeps the input in slices of 256 rows:
// each slice of the feature-major input (256 x 128 fp32, column scales
// applied beforehand) is copied into LDS once per block by direct global ->
// LDS loads, and every synapse of the block's rows with its input in that
// slice reads its row from LDS (LDS serves 16-byte reads at ~121 B/clk/CU).
// The rows' accumulators stay in registers across the slices, so no partial
// sums leave the block and the output is written once, coalesced.
//
// The ULEB128 stream cannot be entered at a slice boundary, so the store
// keeps a derived copy (built on first use, dropped with the structure): per
// synapse its column within its slice (u8), and per row the first synapse
// of every slice.  Value bytes are read from the store itself.
#include "../../include/sili_hip.h"
#include "layer.hpp"
#include "wave.hpp"

#include <algorithm>

namespace sili {

namespace {

constexpr unsigned TPB = 256;
inline unsigned nblk(int64_t n) { return (unsigned)((n + TPB - 1) / TPB); }

constexpr uint32_t SL_W = 256;        // input rows per slice
constexpr uint32_t SL_B = 128;        // batch columns held per LDS row
constexpr uint32_t SL_LD = SL_B;      // LDS row stride in floats (unskewed: 4 groups of 16 lanes reading
                                      // random rows get ~121 B/clk/CU of LDS, a 16-byte skew ~90)
constexpr uint32_t SL_RW = 8;         // output rows per wave
constexpr uint32_t SL_WAVES = 16;     // waves per block
constexpr uint32_t SL_R = SL_RW * SL_WAVES;  // output rows per block
constexpr uint32_t SL_T = SL_WAVES * 64;     // threads per block

// slc_col[e] = column of synapse e within its slice.
__global__ void k_slice_cols(const int32_t *__restrict__ cols, int64_t nnz, uint8_t *__restrict__ out) {
    const int64_t e = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (e < nnz) out[e] = (uint8_t)((uint32_t)cols[e] & (SL_W - 1u));
}

// off[r*(S+1) + s] = the first synapse of row r whose column is >= s*SL_W
// (s = S: the row's end).
__global__ void k_slice_offsets(const uint32_t *__restrict__ elem_start, const int32_t *__restrict__ cols,
                                int64_t rows, int64_t S, uint32_t *__restrict__ off) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i >= rows * (S + 1)) return;
    const int64_t r = i / (S + 1), s = i % (S + 1);
    uint32_t lo = elem_start[r], hi = elem_start[r + 1];
    if (s == S) {
        off[i] = hi;
        return;
    }
    const int64_t key = s * (int64_t)SL_W;
    while (lo < hi) {
        const uint32_t mid = lo + ((hi - lo) >> 1);
        if ((int64_t)cols[mid] < key) lo = mid + 1;
        else hi = mid;
    }
    off[i] = lo;
}

// dst[c, b] = src[c, b] * cs[c] (float4 chunks, q4 of them per input row).
__global__ void k_scale_rows(const float4 *__restrict__ src, const float *__restrict__ cs, int64_t q4, int64_t n4,
                             float4 *__restrict__ dst) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i >= n4) return;
    const float f = cs[i / q4];
    float4 v = src[i];
    v.x *= f;
    v.y *= f;
    v.z *= f;
    v.w *= f;
    dst[i] = v;
}

struct StArgs {
    const uint8_t *scol;   // column within the slice, per synapse
    const uint8_t *val;    // value bytes (w << 4 | imp), per synapse
    const uint32_t *off;   // [rows][S + 1]
    int64_t rows, cols, S;
    const float *rs;       // row (output) scales or NULL
    const float *in;       // feature-major input [cols][B], column scales applied
    int64_t B;
    float *out;            // batch-major output [B][out_ld]
    int64_t out_ld;
};

// One block: SL_R output rows, all slices.  Lane (grp = lane / 16, sub =
// lane % 16): entry slot grp of every 4 the wave takes at a time, batch
// columns [4 sub, 4 sub + 4) and [64 + 4 sub, 64 + 4 sub + 4) (each group's
// float4 reads cover 256 contiguous bytes of one input row).  At each slice
// a wave loads the first 64 synapses of each of its rows in the slice (one
// lane each, all 16 byte loads issued before any wait; the column and the
// weight are then packed in one word, the weight's FP4 value having no low
// mantissa bits) while the block's input loads are in flight; then each
// row's synapses are handed to the entry slots by ds_bpermute, one per slot
// per step (two per slot left more slots empty at a row's end: 28 vs 32 slots
// for a slice's ~26 synapses, 7.55 vs 8.47 ms on c4's gate layer).  A slot past the row's count takes LDS row SL_ZERO, which holds
// zeros, with weight 0; a row with more than 64 synapses in a slice reads
// the rest 64 at a time.  Every access is in bounds: slice rows past the
// input are loaded from row 0 and never referenced.
constexpr uint32_t SL_ZERO = SL_W;  // the zero row, after the slice
// fp4_decode without branches (the same bits for every code)
__device__ __forceinline__ uint32_t fp4_bits(uint32_t code) {
    const uint32_t sgn = (code >> 3) & 1u, e = (code >> 1) & 3u, m = code & 1u;
    const uint32_t normal = (sgn << 31) | ((e + 126u) << 23) | (m << 22);
    const uint32_t sub = m ? (0x3F000000u | (sgn << 31)) : (sgn ? 0x7FC00000u : 0u);
    return e ? normal : sub;
}
// The packed entry of synapse e of [e0, e1) (else the zero row, weight 0),
// from its two bytes loaded beforehand (always from an in-bounds index).
__device__ __forceinline__ uint32_t st_pack2(uint32_t e, uint32_t e1, uint32_t colb, uint32_t valb) {
    return e < e1 ? (fp4_bits(valb >> 4) | colb) : SL_ZERO;
}
__device__ __forceinline__ uint32_t st_pack(const StArgs &a, uint32_t e, uint32_t e1) {
    const uint32_t ei = e < e1 ? e : 0u;  // nnz > 0: index 0 is in bounds
    return st_pack2(e, e1, a.scol[ei], a.val[ei]);
}
__global__ __launch_bounds__(SL_WAVES * 64) void k_gather_staged(StArgs a) {
    extern __shared__ __align__(16) float xs[];  // [SL_W][SL_LD] + a zero row; reused for the output
    const uint32_t t = threadIdx.x, wave = t >> 6, lane = t & 63u;
    const uint32_t grp = lane >> 4, sub = lane & 15u;
    const int64_t r0 = (int64_t)blockIdx.x * SL_R;
    const int64_t rw0 = r0 + (int64_t)wave * SL_RW;
    float acc[SL_RW][8];
#pragma unroll
    for (int k = 0; k < (int)SL_RW; ++k)
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[k][i] = 0.0f;
    for (uint32_t i = t; i < SL_LD; i += SL_T) xs[SL_ZERO * SL_LD + i] = 0.0f;
    const uint32_t nq = (uint32_t)(a.B >> 2);  // float4 chunks of an input row
    constexpr uint32_t CHUNKS = SL_W * SL_B * 4u / 1024u;  // 1 KiB chunks of LDS per slice
    for (int64_t s = 0; s < a.S; ++s) {
        // this slice's synapse ranges of the wave's rows (lane k < SL_RW: row k's
        // start; lane SL_RW + k: its end) and their first 64 synapses
        uint32_t bound = 0;
        if (lane < 2u * SL_RW) {
            const int64_t r = rw0 + (lane & (SL_RW - 1u));
            bound = r < a.rows ? a.off[r * (a.S + 1) + s + (lane >= SL_RW ? 1 : 0)] : 0u;
        }
        uint32_t e0[SL_RW], e1[SL_RW], packed[SL_RW], colb[SL_RW], valb[SL_RW];
        // every row's two bytes loaded first, then decoded: one wait, not 16
#pragma unroll
        for (int k = 0; k < (int)SL_RW; ++k) {
            e0[k] = (uint32_t)__builtin_amdgcn_readlane((int)bound, k);
            e1[k] = (uint32_t)__builtin_amdgcn_readlane((int)bound, (int)SL_RW + k);
            const uint32_t e = e0[k] + lane, ei = e < e1[k] ? e : 0u;
            colb[k] = a.scol[ei];
            valb[k] = a.val[ei];
        }
        __syncthreads();  // the previous slice's reads are done
        // stage input rows [s*SL_W, s*SL_W + SL_W) by direct global -> LDS
        // loads, all issued at once: 16 bytes per lane, each wave instruction
        // filling 1 KiB of LDS (two rows of SL_B floats); lanes past the input
        // or the batch read a valid address (row 0) into LDS that no synapse
        // references
        for (uint32_t k = wave; k < CHUNKS; k += SL_WAVES) {
            const uint32_t lrow = 2u * k + (lane >> 5), q = lane & 31u;
            const int64_t gi = s * SL_W + lrow;
            const float *src = (gi < a.cols && q < nq) ? a.in + gi * a.B + q * 4u : a.in;
            __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void *)(xs + k * 256u), 16, 0, 0);
        }
#pragma unroll
        for (int k = 0; k < (int)SL_RW; ++k) packed[k] = st_pack2(e0[k] + lane, e1[k], colb[k], valb[k]);
        __builtin_amdgcn_s_waitcnt(0);  // every counter: the slice has landed in LDS
        __syncthreads();
        const float *xb = xs;
#pragma unroll
        for (int k = 0; k < (int)SL_RW; ++k) {
            for (uint32_t base = e0[k]; base < e1[k]; base += 64u) {
                const uint32_t n = min(64u, e1[k] - base);
                const uint32_t pk = base == e0[k] ? packed[k] : st_pack(a, base + lane, e1[k]);
                // slot grp takes entry j + grp (< 64); the next step's entry is
                // fetched before this step's reads
                uint32_t q0 = (uint32_t)__shfl((int)pk, (int)grp, 64);
                for (uint32_t j = 0; j < n; j += 4u) {
                    const uint32_t p0 = q0;
                    q0 = (uint32_t)__shfl((int)pk, (int)((j + 4u + grp) & 63u), 64);
                    const float *x0 = xb + (p0 & 0x1FFu) * SL_LD + sub * 4u;
                    const float4 a0 = *reinterpret_cast<const float4 *>(x0);
                    const float4 b0 = *reinterpret_cast<const float4 *>(x0 + 64);
                    const float w0 = __builtin_bit_cast(float, p0 & 0xFFFF0000u);
                    acc[k][0] = __builtin_fmaf(w0, a0.x, acc[k][0]);
                    acc[k][1] = __builtin_fmaf(w0, a0.y, acc[k][1]);
                    acc[k][2] = __builtin_fmaf(w0, a0.z, acc[k][2]);
                    acc[k][3] = __builtin_fmaf(w0, a0.w, acc[k][3]);
                    acc[k][4] = __builtin_fmaf(w0, b0.x, acc[k][4]);
                    acc[k][5] = __builtin_fmaf(w0, b0.y, acc[k][5]);
                    acc[k][6] = __builtin_fmaf(w0, b0.z, acc[k][6]);
                    acc[k][7] = __builtin_fmaf(w0, b0.w, acc[k][7]);
                }
            }
        }
    }
    // the 4 entry slots' partial sums, then the row scale
#pragma unroll
    for (int k = 0; k < (int)SL_RW; ++k)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            float v = acc[k][i];
            v += __shfl_xor(v, 16, 64);
            v += __shfl_xor(v, 32, 64);
            acc[k][i] = v;
        }
    __syncthreads();  // xs becomes the output tile [SL_B][SL_R]
    if (grp == 0) {
#pragma unroll
        for (int k = 0; k < (int)SL_RW; ++k) {
            const int64_t r = rw0 + k;
            const float f = (a.rs && r < a.rows) ? a.rs[r] : 1.0f;
            const uint32_t rl = wave * SL_RW + (uint32_t)k;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                xs[(sub * 4u + (uint32_t)i) * SL_R + rl] = acc[k][i] * f;
                xs[(64u + sub * 4u + (uint32_t)i) * SL_R + rl] = acc[k][4 + i] * f;
            }
        }
    }
    __syncthreads();
    const int64_t nr = min<int64_t>((int64_t)SL_R, a.rows - r0);
    for (uint32_t i = t; i < SL_B * SL_R; i += SL_T) {
        const uint32_t b = i / SL_R, rl = i % SL_R;
        if ((int64_t)b < a.B && (int64_t)rl < nr) a.out[(int64_t)b * a.out_ld + r0 + rl] = xs[i];
    }
}

}  // namespace

// Also: at least one synapse per (row, slice) on average -- the slice copy's
// offsets take 4 bytes per (row, slice), and each row pays a fixed cost per
// slice, so a wide and very sparse layer stays on the segment gather.
bool staged_supported(const Layer &L, const DScatter &s, const ScaleView &sc, const float *in, int64_t B, int skip) {
    const int64_t S = (s.cols + SL_W - 1) / SL_W;
    return s.nnz > 0 && s.nnz < (int64_t(1) << 32) && B > 64 && B <= (int64_t)SL_B && B % 4 == 0 &&
           sc.rank == 1 && skip == SKIP_NONE && (reinterpret_cast<uintptr_t>(in) & 15u) == 0 &&
           s.rows * (S + 1) <= s.nnz;
}

void ensure_slices(Layer &L, DScatter &s, hipStream_t st) {
    if (s.slc_w == (int64_t)SL_W) return;
    ProfScope ps("slices", st);
    const int64_t S = (s.cols + SL_W - 1) / SL_W;
    DevBuf<int32_t> cols;
    cols.ensure((size_t)s.nnz + 1);
    launch_decode(s.plan(), ScaleView{nullptr, nullptr, 1}, cols.p, nullptr, nullptr, st);
    s.slc_col.ensure((size_t)s.nnz + 16);
    launch(k_slice_cols, dim3(nblk(s.nnz)), dim3(TPB), 0, st, (const int32_t *)cols.p, s.nnz, s.slc_col.p);
    const int64_t n = s.rows * (S + 1);
    s.slc_off.ensure((size_t)n + 1);
    if (n > 0)
        launch(k_slice_offsets, dim3(nblk(n)), dim3(TPB), 0, st, (const uint32_t *)s.elem_start.p,
               (const int32_t *)cols.p, s.rows, S, s.slc_off.p);
    SILI_HIP(hipGetLastError());
    SILI_HIP(hipStreamSynchronize(st));  // cols is freed on return
    s.slc_w = SL_W;
    s.slc_n = S;
}

// out[b, r] = sum over row r's synapses (c, w): rs[r] * dec(w) * cs[c] * in[c, b]
// for every row r of the store (written, not added).
void launch_gather_staged(Layer &L, DScatter &s, const ScaleView &sc, const float *in, int64_t B, float *out,
                          int64_t out_ld, hipStream_t st) {
    if (s.rows == 0) return;
    if (!staged_supported(L, s, sc, in, B, SKIP_NONE)) throw_error(SILI_ERR_INVALID, "staged gather: unsupported case");
    ensure_slices(L, s, st);
    const float *xin = in;
    if (sc.ent) {  // the column scales applied to a copy of the input
        ProfScope pss("scale_cols", st);
        L.ws_xs.ensure((size_t)(s.cols * B) + 64);
        const int64_t n4 = s.cols * B / 4;
        launch(k_scale_rows, dim3(nblk(n4)), dim3(TPB), 0, st, reinterpret_cast<const float4 *>(in), sc.ent, B / 4,
               n4, reinterpret_cast<float4 *>(L.ws_xs.p));
        xin = L.ws_xs.p;
    }
    ProfScope ps("gather_staged", st);
    StArgs a{s.slc_col.p, s.val.p, s.slc_off.p, s.rows, s.cols, s.slc_n, sc.row, xin, B, out, out_ld};
    const size_t lds = (size_t)(SL_W + 1) * SL_LD * sizeof(float);
    static_assert((size_t)SL_B * SL_R <= (size_t)SL_W * SL_LD, "the output tile must fit beside the zero row");
    SILI_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(&k_gather_staged),
                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    launch(k_gather_staged, dim3((unsigned)((s.rows + SL_R - 1) / SL_R)), dim3(SL_T), (uint32_t)lds, st, a);
    SILI_HIP(hipGetLastError());
}

}  // namespace sili
