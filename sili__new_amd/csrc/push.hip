// push.hip -- the sparse-input forward as the reference computes it: only the
// active (batch row, input row) pairs contribute (sisldo_forward,
// sisldo_ops.hpp:198-551: per batch row, each stored CSR entry (r, x) pushes
// x * W[r, :] into y[b, :]).
//
// The gather formulation (densify X, then every synapse of the shadow store
// loads its input row's batch values) moves nnz * B * 4 bytes through the load
// path whatever the input's sparsity.  Here a block takes one batch row b (or
// a share of its entries): the input's active rows, their synapse ranges and
// a prefix over their lengths go to LDS, then every thread takes synapses of
// that virtual concatenation one at a time -- coalesced loads of a decoded
// column copy and the value bytes -- and adds x * dec(w) * S(r, c) into an LDS
// copy of y[b, :] (LDS float atomics).  The row's result is stored (or added,
// when the batch row is shared by several blocks) in one coalesced pass.
//
// The ULEB128 stream cannot be entered at an arbitrary synapse, so the store
// keeps a derived copy of its decoded columns (u16: an output row that fits a
// block's LDS has fewer than 2^16 columns), built on the first sparse forward
// and dropped with the store.
#include "../../include/sili_hip.h"
#include "layer.hpp"
#include "wave.hpp"

#include <algorithm>

namespace sili {

namespace {

constexpr unsigned PT = 1024;  // threads per push block
constexpr uint32_t PU = 4;     // 64-synapse steps in flight per wave
constexpr unsigned TPB = 256;
inline unsigned nblk(int64_t n) { return (unsigned)((n + TPB - 1) / TPB); }

struct PushArgs {
    const int32_t *xptrs, *xidx;
    const float *xval;
    int64_t n_in, n_out;
    const uint32_t *elem_start;  // canonical store, [n_in + 1]
    const uint16_t *dcol;        // decoded column per synapse
    const uint8_t *val;          // value bytes (w << 4) | imp
    ScaleView sc;                // canonical: row scale of r, entry scale of c
    float *y;                    // [B, n_out], batch-major
    uint32_t S;                  // blocks per batch row
    uint32_t cap;                // active rows per LDS table pass
    int add;                     // 1: add into y, 0: store
};

__device__ __forceinline__ uint64_t block_sum_u64(uint64_t v, uint64_t *s_part) {
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    if (lane == 0u) s_part[wave] = v;
    __syncthreads();
    uint64_t t = 0;
    for (uint32_t w = 0; w < PT / 64u; ++w) t += s_part[w];
    __syncthreads();
    return t;
}

// In-place exclusive scan of s[0, n) (n <= PT * 4 here); s[n] = the total.
__device__ __forceinline__ void block_excl_scan(uint32_t *s, uint32_t n, uint32_t *s_part) {
    const uint32_t t = threadIdx.x, lane = t & 63u, wave = t >> 6;
    // each thread owns 4 consecutive entries
    const uint32_t i0 = 4u * t;
    uint32_t v[4], sum = 0;
#pragma unroll
    for (uint32_t k = 0; k < 4u; ++k) {
        v[k] = i0 + k < n ? s[i0 + k] : 0u;
        sum += v[k];
    }
    const uint32_t incl = wave_incl_scan(sum);
    if (lane == 63u) s_part[wave] = incl;
    __syncthreads();
    uint32_t before = 0, total = 0;
    for (uint32_t w = 0; w < PT / 64u; ++w) {
        const uint32_t p = s_part[w];
        before += w < wave ? p : 0u;
        total += p;
    }
    uint32_t run = before + incl - sum;
#pragma unroll
    for (uint32_t k = 0; k < 4u; ++k) {
        if (i0 + k < n) s[i0 + k] = run;
        run += v[k];
    }
    if (t == 0) s[n] = total;
    __syncthreads();
}

__global__ __launch_bounds__(PT) void k_push_fwd(PushArgs a) {
    extern __shared__ __align__(16) float s_dyn[];
    __shared__ uint64_t s_part64[PT / 64];
    __shared__ uint32_t s_part[PT / 64];
    __shared__ float s_fp4[16];
    const uint32_t t = threadIdx.x;
    const uint32_t cap = a.cap;
    float *s_y = s_dyn;                                                  // [n_out]
    uint32_t *s_row = reinterpret_cast<uint32_t *>(s_y + a.n_out);      // [cap]
    float *s_xv = reinterpret_cast<float *>(s_row + cap);               // [cap]
    uint32_t *s_beg = reinterpret_cast<uint32_t *>(s_xv + cap);         // [cap]
    float *s_rs = reinterpret_cast<float *>(s_beg + cap);               // [cap]: row scale (rank 1)
    uint32_t *s_off = reinterpret_cast<uint32_t *>(s_rs + cap);         // [cap + 1]
    const int64_t b = blockIdx.x / a.S;
    const uint32_t s = blockIdx.x % a.S;
    if (t < 16u) s_fp4[t] = fp4_decode(t);
    for (int64_t c = t; c < a.n_out; c += PT) s_y[c] = 0.0f;
    const int64_t p0 = a.xptrs[b], p1 = a.xptrs[b + 1];
    const uint16_t *dcol = a.dcol;
    // this block's share of the batch row's synapse visits
    uint64_t lo = 0, hi = ~uint64_t(0);
    if (a.S > 1u) {
        uint64_t my = 0;
        for (int64_t i = p0 + t; i < p1; i += PT) {
            const int64_t r = a.xidx[i];
            if (r >= 0 && r < a.n_in) my += a.elem_start[r + 1] - a.elem_start[r];
        }
        const uint64_t T = block_sum_u64(my, s_part64);
        lo = T * s / a.S;
        hi = T * (s + 1u) / a.S;
    }
    __syncthreads();
    uint64_t base = 0;
    for (int64_t c0 = p0; c0 < p1 && base < hi; c0 += cap) {
        const uint32_t n = (uint32_t)min<int64_t>((int64_t)cap, p1 - c0);
        for (uint32_t i = t; i < n; i += PT) {
            const int64_t r = a.xidx[c0 + i];
            const bool ok = r >= 0 && r < a.n_in;  // the host validates; never read out of bounds
            const uint32_t e0 = ok ? a.elem_start[r] : 0u;
            s_row[i] = ok ? (uint32_t)r : 0u;
            s_rs[i] = (ok && a.sc.rank == 1 && a.sc.row) ? a.sc.row[r] : 1.0f;
            s_xv[i] = a.xval[c0 + i];
            s_beg[i] = e0;
            s_off[i] = ok ? a.elem_start[r + 1] - e0 : 0u;
        }
        __syncthreads();
        block_excl_scan(s_off, n, s_part);
        const uint32_t total = s_off[n];
        const uint64_t e_lo = lo > base ? lo - base : 0, e_hi64 = hi - base;
        const uint32_t e_hi = (uint32_t)min<uint64_t>((uint64_t)total, e_hi64);
        if (e_lo < e_hi) {
            // wave w takes a contiguous run of the block's entries, 64 per
            // step (lane l: entry eb + l); the row index moves forward
            // wave-uniformly (broadcast LDS reads), and PU steps' loads are
            // issued before any is used
            const uint32_t wave = t >> 6, lane = t & 63u;
            const uint32_t span = e_hi - (uint32_t)e_lo;
            const uint32_t per = ((span + PT - 1u) / PT) * 64u;  // entries per wave, a multiple of 64
            const uint32_t w0 = (uint32_t)e_lo + wave * per;
            const uint32_t w1 = min(e_hi, w0 + per);
            if (w0 < w1) {
                // the row holding w0: the last i with s_off[i] <= w0
                uint32_t lo_i = 0, hi_i = n;
                while (hi_i - lo_i > 1u) {
                    const uint32_t mid = (lo_i + hi_i) >> 1;
                    if (s_off[mid] <= w0) lo_i = mid;
                    else hi_i = mid;
                }
                uint32_t i = uniform(lo_i);
                for (uint32_t e = w0; e < w1; e += 64u * PU) {
                    uint32_t ri[PU], ent[PU];
                    bool ok[PU];
#pragma unroll
                    for (uint32_t u = 0; u < PU; ++u) {
                        const uint32_t eb = e + 64u * u;
                        const uint32_t my = eb + lane;
                        ok[u] = my < w1;
                        uint32_t li = i;
                        if (eb < w1) {
                            while (s_off[i + 1] <= eb) ++i;  // the row holding eb
                            li = i;
                            // rows that start inside this step's 64 entries
                            const uint32_t lim = min(eb + 64u, w1);
                            for (uint32_t k = i + 1; k < n && s_off[k] < lim; ++k)
                                if (my >= s_off[k]) li = k;
                        }
                        ri[u] = li;
                        ent[u] = ok[u] ? s_beg[li] + (my - s_off[li]) : 0u;
                    }
                    uint32_t col[PU], code[PU];
#pragma unroll
                    for (uint32_t u = 0; u < PU; ++u) {
                        col[u] = dcol[ent[u]];
                        code[u] = a.val[ent[u]];
                    }
#pragma unroll
                    for (uint32_t u = 0; u < PU; ++u) {
                        const float S = a.sc.rank == 1
                                            ? (a.sc.ent ? s_rs[ri[u]] * a.sc.ent[col[u]] : s_rs[ri[u]])
                                            : scale_at(a.sc, s_row[ri[u]], col[u]);
                        const float v = s_xv[ri[u]] * (s_fp4[code[u] >> 4] * S);
                        if (ok[u]) atomicAdd(s_y + col[u], v);
                    }
                }
            }
        }
        base += total;
        __syncthreads();  // the table is rewritten by the next pass
    }
    __syncthreads();
    float *yrow = a.y + b * a.n_out;
    for (int64_t c = t; c < a.n_out; c += PT) {
        const float v = s_y[c];
        if (!a.add) yrow[c] = v;
        else if (__builtin_bit_cast(uint32_t, v) != 0u) atomicAdd(yrow + c, v);  // +0.0 adds nothing
    }
}

__global__ void k_zero_f32(float *__restrict__ p, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i < n) p[i] = 0.0f;
}

__global__ void k_narrow_u16(const int32_t *__restrict__ src, int64_t n, uint16_t *__restrict__ dst) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i < n) dst[i] = (uint16_t)src[i];
}

// LDS bytes of a push block for n_out outputs and a table of cap rows.
size_t push_lds(int64_t n_out, uint32_t cap) { return (size_t)n_out * 4 + (size_t)cap * 20 + 16; }

}  // namespace

bool push_supported(const Layer &L) {
    return L.W.nnz > 0 && L.W.nnz < (int64_t(1) << 32) && L.n_out <= 65536 &&
           push_lds(L.n_out, 512) <= PUSH_LDS_MAX;
}

void ensure_decoded_cols(Layer &L, hipStream_t st) {
    DScatter &W = L.W;
    if (W.dcol_valid) return;
    if (L.n_out > 65536) throw_error(SILI_ERR_INVALID, "decoded u16 columns need n_outputs <= 65536");
    ProfScope ps("decode_cols", st);
    DevBuf<int32_t> tmp;
    tmp.ensure((size_t)W.nnz + 1);
    W.dcol.ensure((size_t)W.nnz * 2 + 16);
    launch_decode(W.plan(), ScaleView{nullptr, nullptr, 1}, tmp.p, nullptr, nullptr, st);
    launch(k_narrow_u16, dim3(nblk(W.nnz)), dim3(TPB), 0, st, (const int32_t *)tmp.p, W.nnz,
           reinterpret_cast<uint16_t *>(W.dcol.p));
    SILI_HIP(hipGetLastError());
    SILI_HIP(hipStreamSynchronize(st));  // tmp is freed on return
    W.dcol_valid = true;
}

void launch_push_fwd(Layer &L, const int32_t *xptrs, const int32_t *xidx, const float *xval, int64_t B,
                     const ScaleView &sc, float *y, bool add, hipStream_t st) {
    if (B <= 0) return;
    if (!push_supported(L)) throw_error(SILI_ERR_INVALID, "push forward: the output row does not fit a block");
    ensure_decoded_cols(L, st);
    // the LDS table: as many active rows as fit beside y's row (<= 4 * PT for the scan)
    const size_t room = PUSH_LDS_MAX - (size_t)L.n_out * 4 - 16;
    const uint32_t cap = (uint32_t)std::min<size_t>(4 * PT, room / 20);
    // blocks per batch row: about one per CU when the batch is small (a
    // block holds up to PUSH_LDS_MAX of LDS: one per CU), at most 16 adding
    // into one output row
    int64_t S_want = (256 + B - 1) / B;
    if (const int e = env_int("SILI_PUSH_S", 0)) S_want = e;  // tuning knob
    const uint32_t S = (uint32_t)std::max<int64_t>(1, std::min<int64_t>(16, S_want));
    PushArgs a{xptrs, xidx, xval, L.n_in, L.n_out, L.W.elem_start.p,
               reinterpret_cast<const uint16_t *>(L.W.dcol.p), L.W.val.p, sc, y, S, cap,
               (add || S > 1) ? 1 : 0};
    if (S > 1 && !add) {
        ProfScope pz("push_zero", st);
        launch(k_zero_f32, dim3(nblk(B * L.n_out)), dim3(TPB), 0, st, y, B * L.n_out);
    }
    const size_t lds = push_lds(L.n_out, cap);
    ProfScope ps("push", st);
    (void)hipFuncSetAttribute(reinterpret_cast<const void *>(&k_push_fwd), hipFuncAttributeMaxDynamicSharedMemorySize,
                              (int)lds);
    launch(k_push_fwd, dim3((unsigned)(B * S)), dim3(PT), (uint32_t)lds, st, a);
    SILI_HIP(hipGetLastError());
}

}  // namespace sili
