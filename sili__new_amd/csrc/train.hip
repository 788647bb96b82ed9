// train.hip -- backward with the optimizer update (learning_rate != 0) on the
// scattered store: per-synapse RMSprop steps on the stored FP4 weight code and
// its importance, re-quantized in place; the scales' own RMSprop / Adam steps.
//
// Semantics: disldo_backward (linear_disldo.hpp:466-2113) with
// RMSpropScalePolicy, no deferred scale write, BoundedRMSpropSynapsePolicy
// and the constants of sili/cpu_backend.cpp:496-528; rounding deterministic
// (SparseLinearLayerDeterministic, sili/cpu_backend.cpp:1007) or stochastic
// with a counter-based generator (the reference's thread-local xorshift
// stream, fp4quant.hpp:180-265, cannot be reproduced across thread counts).
// Every fp32 expression is evaluated as written, no contraction, in the
// reference's order: per synapse the batch steps run in b order; a row's
// gradient sums (fp64) add the synapses in storage order -- at batch 1 this is
// the reference's own summation order.
#include "layer.hpp"
#include "wave.hpp"

#pragma clang fp contract(off)

namespace sili {

namespace {

constexpr unsigned TPB = 256;
constexpr uint32_t WAVES_T = 4;

__device__ __forceinline__ bool finite_f(float v) { return __builtin_isfinite(v); }
// std::max / std::min as the reference calls them (a NaN first operand is
// returned as is).
__device__ __forceinline__ float std_max(float a, float b) { return (a < b) ? b : a; }
__device__ __forceinline__ float std_min(float a, float b) { return (b < a) ? b : a; }

// BoundedRMSpropSynapsePolicy::update_ci (delta_csr_types.hpp:707-712).
__device__ __forceinline__ float bounded_update_ci(float ci, float g, float contrib, float beta2, float mdf,
                                                   float max_ci) {
    const float ema = beta2 * ci + (1.0f - beta2) * (g * g + contrib * contrib);
    const float floor_ = mdf * ci;
    return std_min(std_max(ema, floor_), max_ci);
}
// BoundedRMSpropSynapsePolicy::update_cw (delta_csr_types.hpp:749-758).
__device__ __forceinline__ float bounded_update_cw(float g, float ci, float S, float eff_lr, float eps, bool damp,
                                                   float max_abs_delta) {
    float raw = damp ? (-g * S) / (__builtin_sqrtf(ci) + eps) : (-g * S);
    if (raw > max_abs_delta) raw = max_abs_delta;
    if (raw < -max_abs_delta) raw = -max_abs_delta;
    return eff_lr * raw;
}
// RMSpropScalePolicy::update (delta_csr_types.hpp:413-434); pow_tab[s] =
// powf(beta2, s), computed on the host with the reference's own function.
__device__ __forceinline__ void rmsprop_scale_update(float &scale, float &state, float g_agg, float eff_lr,
                                                     float beta2, float eps, float contrib_agg, uint32_t &step,
                                                     const float *pow_tab) {
    if (!finite_f(g_agg) || !finite_f(contrib_agg)) return;
    const float new_state = beta2 * state + (1.0f - beta2) * (g_agg * g_agg + contrib_agg * contrib_agg);
    if (!finite_f(new_state)) return;
    float state_hat = new_state;
    ++step;
    const float bias_correction = 1.0f - pow_tab[step];
    if (bias_correction > 0.0f) state_hat = new_state / bias_correction;
    if (!finite_f(state_hat)) return;
    const float new_scale = scale - eff_lr * g_agg / (__builtin_sqrtf(state_hat) + eps);
    if (!finite_f(new_scale)) return;
    state = new_state;
    scale = new_scale;
}

// ---- stochastic rounding ------------------------------------------------------
// One 64-bit draw per quantized value: splitmix64 of (call seed, synapse,
// which), sliced the way fp4_quantize_stochastic slices its xorshift64*
// draw (fp4quant.hpp:198-265): top 24 bits -> uniform [0,1), low 22 bits ->
// dither.
__device__ __forceinline__ uint64_t splitmix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
// fp4quant.hpp:238-265, with the draw supplied.
__device__ __forceinline__ uint32_t fp4_encode_stochastic(float v, uint64_t r) {
    constexpr uint32_t HALF_BITS = 0x3F000000u, ONE_BITS = 0x3F800000u, SIX_BITS = 0x40C00000u;
    const uint32_t bits = __builtin_bit_cast(uint32_t, v);
    const uint32_t sign = bits & 0x80000000u, abits = bits & 0x7FFFFFFFu;
    if (abits > 0x7F800000u) return 0u;
    const float u01 = (float)((double)(r >> 40) * (1.0 / 16777216.0));
    uint32_t mag;
    if (abits >= SIX_BITS) {
        mag = 7u;
    } else if (abits < HALF_BITS) {
        const float av = __builtin_bit_cast(float, abits);
        mag = (u01 < av * 2.0f) ? 1u : 0u;
    } else if (abits < ONE_BITS) {
        const float av = __builtin_bit_cast(float, abits);
        mag = (u01 < av * 2.0f - 1.0f) ? 2u : 1u;
    } else {
        uint32_t rounded = abits + (uint32_t)(r & 0x3FFFFFull);
        if (rounded > SIX_BITS) rounded = SIX_BITS;
        mag = ((((rounded >> 23) & 0xFFu) - 126u) << 1) | ((rounded >> 22) & 1u);
    }
    if (mag == 0u) return 0u;
    return (sign ? 8u : 0u) | mag;
}

// The value byte of a synapse from its updated weight code value and its
// importance in stored units: ValueAccessor<FP4BiPacked>::set / set_stochastic
// (fp4quant.hpp:280-467).  Stochastic draws: splitmix64 of (call seed,
// synapse, which).
__device__ __forceinline__ uint32_t requantize(float w, float imp, bool stochastic, uint64_t seed, uint32_t vb) {
    uint32_t wq, iq;
    if (stochastic) {
        const uint64_t base = seed + 2ull * (uint64_t)vb;
        wq = fp4_encode_stochastic(w, splitmix64(base));
        iq = fp4_encode_stochastic(imp, splitmix64(base + 1ull));
    } else {
        wq = fp4_encode(w);
        iq = fp4_encode(imp);
    }
    return (wq << 4) | iq;
}

// Runs t = step(b, x[b], gcol[b]) for b = 0..B-1 in order and adds the sum
// of t over the wave's lanes into rdx[b].  gcol: one lane's column slice of
// the feature-major gradient (lanes read different columns).  With
// B % 4 == 0 the slice is read 8 batch steps at a time as two 16-byte loads,
// the next group's loads issued before the current group's steps, and the 8
// steps' t are summed over the lanes together: each lane writes its 8 to
// sred (512 floats of LDS per wave), each lane then adds one step's values
// of 8 lanes (read in a rotated order so that the wave's 64 reads hit 64
// different banks), and three exchanges combine the 8 groups.
template <typename Step>
__device__ __forceinline__ void batch_steps(const float *__restrict__ gcol, int64_t B, const float *sx, float *rdx,
                                            float *sred, Step &step) {
    const uint32_t lane = __lane_id();
    if ((B & 3) == 0) {
        const float4 *g4 = reinterpret_cast<const float4 *>(gcol);
        const float4 z4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        float4 n0 = g4[0];
        float4 n1 = B > 4 ? g4[1] : z4;
        const uint32_t j = lane & 7u, grp = lane >> 3;
        // lanes' 8 terms of batch steps b0..b0+7 summed into rdx[b0..]
        auto reduce8 = [&](int64_t b0, const float (&t)[8]) {
            float4 *w4 = reinterpret_cast<float4 *>(sred + lane * 8);
            w4[0] = make_float4(t[0], t[1], t[2], t[3]);
            w4[1] = make_float4(t[4], t[5], t[6], t[7]);
            wave_lds_sync();
            float sum = 0.0f;
#pragma unroll
            for (uint32_t i = 0; i < 8; ++i) sum += sred[(grp * 8u + ((i + grp) & 7u)) * 8u + j];
            sum += __shfl_xor(sum, 8, 64);
            sum += __shfl_xor(sum, 16, 64);
            sum += __shfl_xor(sum, 32, 64);
            if (lane < 8u && b0 + lane < B) rdx[b0 + lane] += sum;
            wave_lds_sync();
        };
        const int64_t full = B & ~(int64_t)7;
        for (int64_t b0 = 0; b0 < full; b0 += 8) {
            const float4 c0 = n0, c1 = n1;
            if (b0 + 8 < B) n0 = g4[(b0 + 8) >> 2];
            if (b0 + 12 < B) n1 = g4[(b0 + 12) >> 2];
            const float d[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
            float t[8];
#pragma unroll
            for (int q = 0; q < 8; ++q) t[q] = step(b0 + q, sx[b0 + q], d[q]);
            reduce8(b0, t);
        }
        if (B & 4) {  // last 4 steps (loaded by the last full group, or up front)
            const float d[4] = {n0.x, n0.y, n0.z, n0.w};
            float t[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int q = 0; q < 4; ++q) t[q] = step(full + q, sx[full + q], d[q]);
            reduce8(full, t);
        }
    } else {
        for (int64_t b = 0; b < B; ++b) {
            const float tot = wave_sum(step(b, sx[b], gcol[b]));
            if (lane == 0u) rdx[b] = rdx[b] + tot;
        }
    }
}

struct TrainArgs {
    const uint32_t *byte_start, *elem_start;  // canonical store
    const uint8_t *idx;
    uint8_t *val;
    int64_t n_in, n_out;
    int64_t B;
    const float *xT, *gT;      // feature-major [n_in][B], [n_out][B]
    float *dx;                 // [B][n_in], overwritten
    float *vs, *vs_imp;        // [n_in*rank]
    uint32_t *vs_step;
    const float *os;           // [n_out*rank]
    const float *is, *ois;     // importance scales (NULL: ones)
    const float *pow_tab;
    float *mterm;              // [nnz * 2 * rank] column-gradient terms, or NULL
    const float *vs_read;      // the scales the rows read (a snapshot when rows write others' slots)
    float *def_w, *def_i;      // DeferredScaleWrite: true-units weight and importance per synapse
    float lr, beta2, eps, min_decay_frac, max_abs_delta, max_ci, zero_escape_eps;
    int lr_per_row_nnz, damp, stochastic;
    int deferred, no_scale;    // DeferredScaleWrite; NoScalePolicy
    uint64_t seed;             // this call's stochastic-rounding seed
};

// One wave per canonical row (linear_disldo.hpp:624-880).  The row's entries
// are decoded 64 index bytes at a time; each lane owns one entry and runs its
// batch steps; the row's fp64 gradient sums are added by lane 0 in entry
// order; dx[b][row] is the sum over the row's entries of the updated weight
// times dy, reduced across the lanes per b.
//   scales written in the loop (default): the stored code value `quant` is
//     stepped by dL/dquant = g * S(row, col), re-quantized in place; scale
//     gradients weigh each term by quant (0.1 for an exact zero), per
//     component (linear_disldo.hpp:791-896);
//   DeferredScaleWrite: the true-units weight cw = code * vs0 * os0 is
//     stepped by g; scale gradients weigh by the stored code, component 0
//     only; (cw, ci) are kept for k_train_store (linear_disldo.hpp:687-790).
template <int RANK, bool DEFERRED, bool COLS>
__global__ __launch_bounds__(256) void k_train_rows(TrainArgs a) {
    __shared__ double s_part[WAVES_T][64][2 * RANK];
    extern __shared__ __attribute__((aligned(16))) float s_dyn[];  // [wave][dx B | x B]
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const int64_t r = (int64_t)blockIdx.x * WAVES_T + wave;
    if (r >= a.n_in) return;
    const uint32_t e0 = a.elem_start[r], e1 = a.elem_start[r + 1];
    const uint32_t nnz = e1 - e0;
    const int64_t B = a.B;
    if (nnz == 0) {
        for (int64_t b = lane; b < B; b += 64) a.dx[b * a.n_in + r] = 0.0f;
        return;
    }
    float *rdx = s_dyn + (int64_t)wave * (2 * B + 512);
    float *sx = rdx + B;       // the row's inputs, read by every lane
    float *sred = sx + B;      // dx reduction staging (batch_steps)
    const float *xrow = a.xT + r * B;
    for (int64_t b = lane; b < B; b += 64) {
        rdx[b] = 0.0f;
        sx[b] = xrow[b];
    }
    wave_lds_sync();
    const float eff_lr = a.lr_per_row_nnz ? a.lr / (float)nnz : a.lr;
    const float scale_eff_lr = a.lr / (float)nnz;
    const float imp_scale = a.is ? a.is[r] : 1.0f;
    float vs_k[RANK];
#pragma unroll
    for (int k = 0; k < RANK; ++k) vs_k[k] = a.vs_read[r * RANK + k];
    constexpr bool deferred = DEFERRED;
    constexpr int nk = DEFERRED ? 1 : RANK;  // components that take gradient terms
    double sg[RANK], sgc[RANK];
#pragma unroll
    for (int k = 0; k < RANK; ++k) sg[k] = sgc[k] = 0.0;
    uint32_t pos = a.byte_start[r], carry = 0, ebase = e0;
    const uint32_t end = a.byte_start[r + 1];
    while (pos < end) {
        const Chunk ch = decode_chunk(a.idx, pos, end, carry);
        if (ch.T == 0ull) break;
        const bool has = ch.term;
        const uint32_t col = has ? ch.col : 0u;
        const uint32_t vb = ebase + ch.rank;
        const uint32_t byte = has ? (uint32_t)a.val[vb] : 0u;
        const float cw_orig = fp4_decode(byte >> 4);
        const float ci_orig = fp4_decode(byte & 0xFu);
        const float out_imp_scale = (a.ois && has) ? a.ois[col] : 1.0f;
        const float combined_imp_scale = imp_scale * out_imp_scale;
        float ci = ci_orig * combined_imp_scale;
        float os_k[RANK];
        float S = 0.0f;
#pragma unroll
        for (int k = 0; k < RANK; ++k) {
            os_k[k] = has ? a.os[(int64_t)col * RANK + k] : 0.0f;
            S = S + vs_k[k] * os_k[k];
        }
        // wv: the stepped weight (code units; true units when deferred)
        const float S_step = deferred ? 1.0f : S;
        float wv = deferred ? cw_orig * (vs_k[0] * os_k[0]) : cw_orig;
        float cw = deferred ? wv : wv * S;
        double psg[RANK], psgc[RANK];
        float pm[RANK], pmc[RANK];
#pragma unroll
        for (int k = 0; k < RANK; ++k) {
            psg[k] = psgc[k] = 0.0;
            pm[k] = pmc[k] = 0.0f;
        }
        // one batch step of this lane's synapse (b in order); lanes without
        // a synapse step zeros (finite throughout) and contribute nothing
        auto step = [&](int64_t b, float iv, float dy_raw) -> float {
            const float dyv = has ? dy_raw : 0.0f;
            const float g = dyv * iv;
            {
                const float contrib = iv * cw_orig;
                ci = bounded_update_ci(ci, g, contrib, a.beta2, a.min_decay_frac, a.max_ci);
                wv = wv + bounded_update_cw(g, ci, S_step, eff_lr, a.eps, a.damp != 0, a.max_abs_delta);
                cw = deferred ? wv : wv * S;
                const float qf = deferred ? cw_orig : ((wv == 0.0f) ? a.zero_escape_eps : wv);
#pragma unroll
                for (int k = 0; k < nk; ++k) {
                    psg[k] = psg[k] + ((double)qf * (double)os_k[k]) * (double)g;
                    psgc[k] = psgc[k] + ((double)qf * (double)os_k[k]) * (double)contrib;
                    if constexpr (COLS) {
                        pm[k] = pm[k] + (qf * vs_k[k]) * g;
                        pmc[k] = pmc[k] + (qf * vs_k[k]) * contrib;
                    }
                }
            }
            // dx[b][row]: this synapse's term
            return has ? cw * dyv : 0.0f;
        };
        batch_steps(a.gT + (int64_t)col * B, B, sx, rdx, sred, step);
        if (has) {
            if (deferred) {
                a.def_w[vb] = wv;
                a.def_i[vb] = ci;
            } else {
                a.val[vb] = (uint8_t)requantize(wv, ci / combined_imp_scale, a.stochastic != 0, a.seed, vb);
            }
            if constexpr (COLS) {
#pragma unroll
                for (int k = 0; k < RANK; ++k) {
                    a.mterm[(int64_t)vb * 2 * RANK + k] = pm[k];
                    a.mterm[(int64_t)vb * 2 * RANK + RANK + k] = pmc[k];
                }
            }
        }
        // the row's gradient sums, entry by entry in storage order
#pragma unroll
        for (int k = 0; k < RANK; ++k) {
            s_part[wave][lane][k] = has ? psg[k] : 0.0;
            s_part[wave][lane][RANK + k] = has ? psgc[k] : 0.0;
        }
        wave_lds_sync();
        if (lane == 0u) {
            uint64_t T = ch.T;
            while (T) {
                const uint32_t l = (uint32_t)__builtin_ctzll(T);
                T &= T - 1ull;
#pragma unroll
                for (int k = 0; k < RANK; ++k) {
                    sg[k] = sg[k] + s_part[wave][l][k];
                    sgc[k] = sgc[k] + s_part[wave][l][RANK + k];
                }
            }
        }
        wave_lds_sync();
        carry = chunk_advance(ch, pos, ebase);
    }
    wave_lds_sync();
    for (int64_t b = lane; b < B; b += 64) a.dx[b * a.n_in + r] = rdx[b];
    // the row's scale step (linear_disldo.hpp:898-925)
    if (lane == 0u && !a.no_scale) {
#pragma unroll
        for (int k = 0; k < nk; ++k) {
            // DeferredScaleWrite indexes the scale and its second moment by
            // the row alone (slot r: component r % rank of row r / rank once
            // rank > 1) and its step counter by (r, 0)
            const int64_t i = deferred ? r : r * RANK + k;
            const int64_t is_ = r * RANK + k;
            float vsv = a.vs[i], st = a.vs_imp[i];
            uint32_t step = a.vs_step[is_];
            rmsprop_scale_update(vsv, st, (float)sg[k], scale_eff_lr, a.beta2, a.eps, (float)sgc[k], step, a.pow_tab);
            a.vs[i] = vsv;
            a.vs_imp[i] = st;
            a.vs_step[is_] = step;
        }
    }
}

// DeferredScaleWrite's store (linear_disldo.hpp:2090-2112): every synapse's
// (cw, ci) re-quantized under the scales in effect after the call, one wave
// per canonical row.
template <int RANK>
__global__ __launch_bounds__(256) void k_train_store(TrainArgs a) {
    const uint32_t wave = threadIdx.x >> 6;
    const int64_t r = (int64_t)blockIdx.x * WAVES_T + wave;
    if (r >= a.n_in) return;
    const uint32_t e0 = a.elem_start[r], e1 = a.elem_start[r + 1];
    if (e1 == e0) return;
    const float fvs = a.vs[r * RANK];
    const float fis = a.is ? a.is[r] : 1.0f;
    uint32_t pos = a.byte_start[r], carry = 0, ebase = e0;
    const uint32_t end = a.byte_start[r + 1];
    while (pos < end) {
        const Chunk ch = decode_chunk(a.idx, pos, end, carry);
        if (ch.T == 0ull) break;
        if (ch.term) {
            const uint32_t vb = ebase + ch.rank;
            const float fos = a.os[(int64_t)ch.col * RANK];
            const float fois = a.ois ? a.ois[ch.col] : 1.0f;
            const float final_combined_scale = fvs * fos;
            const float final_combined_imp_scale = fis * fois;
            a.val[vb] = (uint8_t)requantize(a.def_w[vb] / final_combined_scale,
                                            a.def_i[vb] / final_combined_imp_scale, a.stochastic != 0, a.seed, vb);
        }
        carry = chunk_advance(ch, pos, ebase);
    }
}

// ---- backward_sparse with the optimizer update ------------------------------------
struct SparseTrainArgs {
    const uint32_t *byte_start, *elem_start;  // canonical store
    const uint8_t *idx;
    uint8_t *val;
    int64_t n_in, B;
    const float *xT;         // [n_in][B]
    const float *gT;         // [n_out][B], +0.0 where dy has no entry, explicit entries nonzero bits
    float *dx;               // [B][n_in], overwritten
    const float *vs, *os;    // [n*rank]; component 0 is read
    const float *is, *ois;   // importance scales (NULL: ones)
    double *rowsum;          // [n_in][2]: the row's value-scale gradient sums
    int rank;
    float lr, beta2, eps;
    int lr_per_row_nnz, damp;
};

// One wave per canonical row (sisldo_ops.hpp:637-729): each lane owns one
// synapse and takes the batch rows in order; at every batch row whose dy
// holds the synapse's column, the weight and importance are stepped in true
// units and stored back (round to nearest), so the next batch row reads the
// re-quantized code.  No bound on the importance EMA or the step.
__global__ __launch_bounds__(256) void k_sparse_train_rows(SparseTrainArgs a) {
    __shared__ double s_part[WAVES_T][64][2];
    extern __shared__ __attribute__((aligned(16))) float s_dyn[];  // [wave][dx B | x B]
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const int64_t r = (int64_t)blockIdx.x * WAVES_T + wave;
    if (r >= a.n_in) return;
    const uint32_t e0 = a.elem_start[r], e1 = a.elem_start[r + 1];
    const int64_t B = a.B;
    if (e1 == e0) {
        for (int64_t b = lane; b < B; b += 64) a.dx[b * a.n_in + r] = 0.0f;
        if (lane == 0u) a.rowsum[2 * r] = a.rowsum[2 * r + 1] = 0.0;
        return;
    }
    float *rdx = s_dyn + (int64_t)wave * (2 * B + 512);
    float *sx = rdx + B;
    float *sred = sx + B;
    const float *xrow = a.xT + r * B;
    for (int64_t b = lane; b < B; b += 64) {
        rdx[b] = 0.0f;
        sx[b] = xrow[b];
    }
    wave_lds_sync();
    const float eff_lr = a.lr_per_row_nnz ? a.lr / (float)(e1 - e0) : a.lr;
    const float imp_scale = a.is ? a.is[r] : 1.0f;
    const float val_scale = a.vs[r * a.rank];
    double sg = 0.0, sgc = 0.0;
    uint32_t pos = a.byte_start[r], carry = 0, ebase = e0;
    const uint32_t end = a.byte_start[r + 1];
    while (pos < end) {
        const Chunk ch = decode_chunk(a.idx, pos, end, carry);
        if (ch.T == 0ull) break;
        const bool has = ch.term;
        const uint32_t col = has ? ch.col : 0u;
        const uint32_t vb = ebase + ch.rank;
        uint32_t byte = has ? (uint32_t)a.val[vb] : 0u;
        const float out_scale = has ? a.os[(int64_t)col * a.rank] : 0.0f;
        const float combined_scale = val_scale * out_scale;
        const float out_imp_scale = (a.ois && has) ? a.ois[col] : 1.0f;
        const float combined_imp_scale = imp_scale * out_imp_scale;
        double psg = 0.0, psgc = 0.0;
        // lanes whose synapse has no dy entry at b compute and discard
        auto step = [&](int64_t b, float iv, float dy_raw) -> float {
            const float dyv = has ? dy_raw : 0.0f;
            const bool present = __builtin_bit_cast(uint32_t, dyv) != 0u;
            const float w_stored = fp4_decode(byte >> 4);
            const float w = w_stored * combined_scale;
            const float grad = dyv * iv;
            float imp = fp4_decode(byte & 0xFu) * combined_imp_scale;
            const float contrib = iv * w;
            imp = a.beta2 * imp + (1.0f - a.beta2) * (grad * grad + contrib * contrib);
            const float new_w = w + (a.damp ? (-eff_lr * grad) / (__builtin_sqrtf(imp) + a.eps) : (-eff_lr * grad));
            const uint32_t nb = (fp4_encode(new_w / combined_scale) << 4) | fp4_encode(imp / combined_imp_scale);
            byte = present ? nb : byte;
            psg = psg + (present ? ((double)w_stored * (double)out_scale) * (double)grad : 0.0);
            psgc = psgc + (present ? ((double)w_stored * (double)out_scale) * (double)contrib : 0.0);
            return present ? w * dyv : 0.0f;
        };
        batch_steps(a.gT + (int64_t)col * B, B, sx, rdx, sred, step);
        if (has) a.val[vb] = (uint8_t)byte;
        s_part[wave][lane][0] = has ? psg : 0.0;
        s_part[wave][lane][1] = has ? psgc : 0.0;
        wave_lds_sync();
        if (lane == 0u) {
            uint64_t T = ch.T;
            while (T) {
                const uint32_t l = (uint32_t)__builtin_ctzll(T);
                T &= T - 1ull;
                sg = sg + s_part[wave][l][0];
                sgc = sgc + s_part[wave][l][1];
            }
        }
        wave_lds_sync();
        carry = chunk_advance(ch, pos, ebase);
    }
    wave_lds_sync();
    for (int64_t b = lane; b < B; b += 64) a.dx[b * a.n_in + r] = rdx[b];
    if (lane == 0u) {
        a.rowsum[2 * r] = sg;
        a.rowsum[2 * r + 1] = sgc;
    }
}

// value_scale's step after all batch rows (sisldo_ops.hpp:820-846): slot r of
// the scale and its second moment, step counter (r, 0), no finiteness guard.
__global__ __launch_bounds__(256) void k_sparse_train_vs(const uint32_t *__restrict__ elem_start, int64_t n_in,
                                                         int rank, const double *__restrict__ rowsum, float *vs,
                                                         float *vs_imp, uint32_t *vs_step, float lr, float beta2,
                                                         float eps, const float *__restrict__ pow_tab) {
    const int64_t r = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (r >= n_in) return;
    const double s = rowsum[2 * r], sc = rowsum[2 * r + 1];
    if (s == 0.0 && sc == 0.0) return;
    const uint32_t nnz = elem_start[r + 1] - elem_start[r];
    if (nnz == 0) return;
    const float scale_eff_lr = lr / (float)nnz;
    const float g_agg = (float)s, contrib_agg = (float)sc;
    const float new_vs_imp = beta2 * vs_imp[r] + (1.0f - beta2) * (g_agg * g_agg + contrib_agg * contrib_agg);
    const uint32_t step = vs_step[r * rank] + 1u;
    vs_step[r * rank] = step;
    const float bias_correction = 1.0f - pow_tab[step];
    const float vs_imp_hat = bias_correction > 0.0f ? new_vs_imp / bias_correction : new_vs_imp;
    vs_imp[r] = new_vs_imp;
    vs[r] = vs[r] - scale_eff_lr * g_agg / (__builtin_sqrtf(vs_imp_hat) + eps);
}

// ---- block4 tiles ------------------------------------------------------------------
struct B4TrainArgs {
    const uint32_t *byte_start, *tile_start;  // canonical block4 store
    const uint8_t *idx;
    uint8_t *tiles;
    int64_t brows, n_in, n_out, B, nnz_scattered;
    const float *xT, *gT;
    float *dx;                 // [B][n_in], added into
    float *vs, *vs_imp;
    uint32_t *vs_step;
    const float *os, *is, *ois, *pow_tab;
    float *b4term;             // [tiles * 16][2 * rank] or NULL
    float lr, beta2, eps, min_decay_frac, max_abs_delta, max_ci, zero_escape_eps;
    int lr_per_row_nnz, damp, stochastic;
    uint64_t seed;
};

// One wave per canonical block row (linear_disldo.hpp:962-1951, FP4): every
// slot of the row's tiles trains.  Lanes hold 4 tiles x 16 slots, ordered
// (tile, li, lj) so a quad is one tile row.  A tile whose 4 columns are all
// in range sums its row's 4 row-gradient and dx terms per batch step in lane
// order ((t0 + t1) + t2) + t3 in fp32 (the reference's 4-lane path); an
// edge tile adds its fp64 row-gradient terms one by one (its scalar path).
// The tiles' fp64 row partials are added in tile order; then the block
// rows' scale step.
// Lane J of the calling lane's quad (DPP quad_perm, a VALU move).
template <int J>
__device__ __forceinline__ float quad_lane(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), J * 0x55, 0xF, 0xF, false));
}
template <int J>
__device__ __forceinline__ double quad_lane(double v) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)u, J * 0x55, 0xF, 0xF, false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)(u >> 32), J * 0x55, 0xF, 0xF, false);
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}
// ((l0 + l1) + l2) + l3 over the quad, on every lane of it
template <typename T>
__device__ __forceinline__ T quad_sum(T v) {
    return ((quad_lane<0>(v) + quad_lane<1>(v)) + quad_lane<2>(v)) + quad_lane<3>(v);
}

constexpr uint32_t WAVES_B4 = 2;  // waves per block of k_train_b4 (LDS: 4 rows x B floats per wave)

template <int RANK>
__global__ __launch_bounds__(128) void k_train_b4(B4TrainArgs a) {
    __shared__ uint32_t s_bc[WAVES_B4][64];
    __shared__ double s_mr[WAVES_B4][4][4][2 * RANK];  // [tile][li][k | contrib k]
    extern __shared__ float s_dxb[];                    // [wave][li][B]: the block row's dx terms
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const int64_t br = (int64_t)blockIdx.x * WAVES_B4 + wave;
    if (br >= a.brows) return;
    const uint32_t t0 = a.tile_start[br], t1 = a.tile_start[br + 1];
    if (t0 == t1) return;
    const int64_t B = a.B;
    float *sdx = s_dxb + (int64_t)wave * 4 * B;
    for (int64_t i = lane; i < 4 * B; i += 64) sdx[i] = 0.0f;
    wave_lds_sync();
    const uint32_t nnz_row = (t1 - t0) * 4u;
    const float eff_lr = a.lr_per_row_nnz ? a.lr / (float)nnz_row : a.lr;
    const uint32_t tl = lane >> 4, li = (lane >> 2) & 3u, lj = lane & 3u;
    const int64_t row = br * 4 + li;
    const bool row_ok = row < a.n_in;
    double rowacc[2 * RANK];  // lanes 0..3: row br*4 + lane
#pragma unroll
    for (int k = 0; k < 2 * RANK; ++k) rowacc[k] = 0.0;
    uint32_t pos = a.byte_start[br], carry = 0, ebase = t0;
    const uint32_t end = a.byte_start[br + 1];
    while (pos < end) {
        const Chunk ch = decode_chunk(a.idx, pos, end, carry);
        if (ch.T == 0ull) break;
        if (ch.term) s_bc[wave][ch.rank] = ch.col;
        wave_lds_sync();
        const uint32_t nt = (uint32_t)__popcll(ch.T);
        for (uint32_t sub = 0; sub < nt; sub += 4) {
            const uint32_t trank = sub + tl;
            const bool tile_ok = trank < nt;
            const uint32_t bc = tile_ok ? s_bc[wave][trank] : 0u;
            const int64_t t = (int64_t)ebase + trank;
            const int64_t col = (int64_t)bc * 4 + lj;
            const bool has = tile_ok && row_ok && col < a.n_out;
            const bool full = tile_ok && (int64_t)bc * 4 + 4 <= a.n_out;
            const uint32_t slot = lj * 4u + li;
            const uint32_t byte = has ? (uint32_t)a.tiles[t * 16 + slot] : 0u;
            float vs_k[RANK], os_k[RANK];
            float S = 0.0f;
#pragma unroll
            for (int k = 0; k < RANK; ++k) {
                vs_k[k] = row_ok ? a.vs[row * RANK + k] : 0.0f;
                os_k[k] = has ? a.os[col * RANK + k] : 0.0f;
                S = S + vs_k[k] * os_k[k];
            }
            const float imp_scale = (a.is && row_ok) ? a.is[row] : 1.0f;
            const float cis = imp_scale * ((a.ois && has) ? a.ois[col] : 1.0f);
            const float q0 = fp4_decode(byte & 0xFu);
            float q = q0;
            float ci = fp4_decode(byte >> 4) * cis;
            double mr[2 * RANK];
            float mc[2 * RANK];
#pragma unroll
            for (int k = 0; k < 2 * RANK; ++k) {
                mr[k] = 0.0;
                mc[k] = 0.0f;
            }
            const float *xrow = a.xT + (row_ok ? row : 0) * B;
            const float *gcol = a.gT + (has ? col : 0) * B;
            // one batch step of this lane's slot (b in order)
            auto step = [&](int64_t b, float iv_raw, float dy_raw) {
                const float iv = row_ok ? iv_raw : 0.0f;
                const float dyv = has ? dy_raw : 0.0f;
                const float g = dyv * iv;
                const float contrib = q0 * iv;
                ci = bounded_update_ci(ci, g, contrib, a.beta2, a.min_decay_frac, a.max_ci);
                q = q + bounded_update_cw(g, ci, S, eff_lr, a.eps, a.damp != 0, a.max_abs_delta);
                const float qf = (q == 0.0f) ? a.zero_escape_eps : q;
                const float tdx = has ? (q * S) * dyv : 0.0f;
#pragma unroll
                for (int k = 0; k < RANK; ++k) {
                    mc[k] = mc[k] + (qf * vs_k[k]) * g;
                    mc[RANK + k] = mc[RANK + k] + (qf * vs_k[k]) * contrib;
                }
                // the tile row's 4 dx terms, summed on the quad, into the
                // block row's LDS row (4 tiles of a pass add to one address)
                const float qdx = quad_sum(tdx);
                if (lj == 0u && tile_ok) atomicAdd(&sdx[(int64_t)li * B + b], qdx);
                // a quad is one tile row: full is uniform over it
                if (full) {
#pragma unroll
                    for (int k = 0; k < RANK; ++k) {
                        mr[k] = mr[k] + (double)quad_sum((qf * os_k[k]) * g);
                        mr[RANK + k] = mr[RANK + k] + (double)quad_sum((qf * os_k[k]) * contrib);
                    }
                } else {
#pragma unroll
                    for (int k = 0; k < RANK; ++k) {
                        const double d0 = has ? ((double)qf * (double)os_k[k]) * (double)g : 0.0;
                        const double d1 = has ? ((double)qf * (double)os_k[k]) * (double)contrib : 0.0;
                        mr[k] = (((mr[k] + quad_lane<0>(d0)) + quad_lane<1>(d0)) + quad_lane<2>(d0)) + quad_lane<3>(d0);
                        mr[RANK + k] =
                            (((mr[RANK + k] + quad_lane<0>(d1)) + quad_lane<1>(d1)) + quad_lane<2>(d1)) + quad_lane<3>(d1);
                    }
                }
            };
            int64_t b = 0;
            if ((B & 3) == 0) {
                // 4 batch steps per pair of 16-byte loads (rows are B floats, B % 4 == 0)
                for (; b < B; b += 4) {
                    const float4 xv = *reinterpret_cast<const float4 *>(xrow + b);
                    const float4 gv = *reinterpret_cast<const float4 *>(gcol + b);
                    step(b, xv.x, gv.x);
                    step(b + 1, xv.y, gv.y);
                    step(b + 2, xv.z, gv.z);
                    step(b + 3, xv.w, gv.w);
                }
            }
            for (; b < B; ++b) step(b, xrow[b], gcol[b]);
            if (has) {
                const float imp = ci / cis;
                uint32_t wq, iq;
                if (a.stochastic) {
                    const uint64_t base = a.seed + 2ull * (uint64_t)(a.nnz_scattered + t * 16 + slot);
                    wq = fp4_encode_stochastic(q, splitmix64(base));
                    iq = fp4_encode_stochastic(imp, splitmix64(base + 1ull));
                } else {
                    wq = fp4_encode(q);
                    iq = fp4_encode(imp);
                }
                a.tiles[t * 16 + slot] = (uint8_t)((iq << 4) | wq);
                if (a.b4term) {
#pragma unroll
                    for (int k = 0; k < 2 * RANK; ++k) a.b4term[(t * 16 + slot) * 2 * RANK + k] = mc[k];
                }
            }
            // the tile rows' fp64 partials, added per row in tile order
            if (lj == 0u) {
#pragma unroll
                for (int k = 0; k < 2 * RANK; ++k) s_mr[wave][tl][li][k] = tile_ok ? mr[k] : 0.0;
            }
            wave_lds_sync();
            if (lane < 4u) {
                for (uint32_t u = 0; u < 4u && sub + u < nt; ++u) {
#pragma unroll
                    for (int k = 0; k < 2 * RANK; ++k) rowacc[k] = rowacc[k] + s_mr[wave][u][lane][k];
                }
            }
            wave_lds_sync();
        }
        carry = chunk_advance(ch, pos, ebase);
    }
    wave_lds_sync();
    for (uint32_t l = 0; l < 4u; ++l) {
        const int64_t rr = br * 4 + l;
        if (rr >= a.n_in) break;
        for (int64_t b = lane; b < B; b += 64) a.dx[b * a.n_in + rr] += sdx[(int64_t)l * B + b];
    }
    // the block rows' scale step (linear_disldo.hpp:1923-1951)
    const int64_t r = br * 4 + lane;
    if (lane < 4u && r < a.n_in) {
        const float scale_eff_lr = a.lr / (float)nnz_row;
#pragma unroll
        for (int k = 0; k < RANK; ++k) {
            const double sum = rowacc[k], sum_c = rowacc[RANK + k];
            if (sum == 0.0 && sum_c == 0.0) continue;
            const float g_agg = (float)sum, contrib_agg = (float)sum_c;
            if (!finite_f(g_agg) || !finite_f(contrib_agg)) continue;
            const int64_t i = r * RANK + k;
            const float new_vs_imp = a.beta2 * a.vs_imp[i] + (1.0f - a.beta2) * (g_agg * g_agg + contrib_agg * contrib_agg);
            if (!finite_f(new_vs_imp)) continue;
            const uint32_t step = a.vs_step[i] + 1u;
            a.vs_step[i] = step;
            const float bias_correction = 1.0f - a.pow_tab[step];
            const float hat = bias_correction > 0.0f ? new_vs_imp / bias_correction : new_vs_imp;
            if (!finite_f(hat)) continue;
            const float new_vs = a.vs[i] - scale_eff_lr * g_agg / (__builtin_sqrtf(hat) + a.eps);
            if (!finite_f(new_vs)) continue;
            a.vs_imp[i] = new_vs_imp;
            a.vs[i] = new_vs;
        }
    }
}

// ---- the block rows' write-back with eviction --------------------------------
// Block4Store::merge_row_workspace (block4.hpp:1367-1462) for one block row,
// tiles t0..t1 (canonical order, tcol[t] the tile's block column), by one
// wave: every lane calls it with the same arguments.  used: the row's stored
// bytes (tiles sparse-packed or 16 bytes by flags[t]), alloc: its reserved
// tile bytes.  While the row does not fit, its live slot of lowest
// |importance code x is[row] x ois[col]| (fp64) is zeroed -- in the
// reference's scan order (tile, tile row, tile column), the first on ties;
// a NaN importance met first is never displaced -- and its tile re-encoded by
// live count.  A row that still does not fit counts an overflow event and
// the bytes past its last whole tile that fits.  Tile words are read and
// written at device scope (they are rewritten while other lanes scan them);
// lane 0 makes every write.  ctr: [evicted, overflow events, overflow bytes].
__device__ __forceinline__ uint32_t tile_word_load(const uint8_t *tiles, uint64_t w) {
    return __hip_atomic_load(reinterpret_cast<const uint32_t *>(tiles) + w, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t word_live(uint32_t v) {
    return (uint32_t)((v & 0xFFu) != 0u) + (uint32_t)((v & 0xFF00u) != 0u) + (uint32_t)((v & 0xFF0000u) != 0u) +
           (uint32_t)((v & 0xFF000000u) != 0u);
}

__device__ void b4_merge_row_wave(uint8_t *tiles, uint8_t *flags, const uint32_t *__restrict__ tcol, uint32_t t0,
                                  uint32_t t1, int64_t br, uint64_t used, uint64_t alloc, const float *is,
                                  const float *ois, int64_t n_in, int64_t n_out, uint32_t sp,
                                  unsigned long long *ctr) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t npos = (t1 - t0) * 16u;
    while (used > alloc) {
        uint32_t first = 0xFFFFFFFFu, bp = 0xFFFFFFFFu;
        double first_a = 0.0, ba = 0.0;
        for (uint32_t p = lane; p < npos; p += 64u) {
            const uint32_t t = t0 + (p >> 4), li = (p >> 2) & 3u, lj = p & 3u, slot = lj * 4u + li;
            const uint32_t v = tile_word_load(tiles, (uint64_t)t * 4u + (slot >> 2));
            const uint32_t byte = (v >> (8u * (slot & 3u))) & 0xFFu;
            if (byte == 0u) continue;
            const int64_t row = br * 4 + li, col = (int64_t)tcol[t] * 4 + lj;
            const float isv = (is && row < n_in) ? is[row] : 1.0f;
            const float oisv = (ois && col < n_out) ? ois[col] : 1.0f;
            const double a = __builtin_fabs((double)fp4_decode(byte >> 4) * (double)isv * (double)oisv);
            if (p < first) {
                first = p;
                first_a = a;
            }
            if (!__builtin_isnan(a) && (bp == 0xFFFFFFFFu || a < ba || (a == ba && p < bp))) {
                ba = a;
                bp = p;
            }
        }
        // wave minima: the first live slot, and the lowest (|imp|, position)
        // over the slots whose importance is a number
        for (int off = 32; off >= 1; off >>= 1) {
            const uint32_t of = (uint32_t)__shfl_xor((int)first, off);
            const double ofa = __shfl_xor(first_a, off);
            if (of < first) {
                first = of;
                first_a = ofa;
            }
            const uint32_t obp = (uint32_t)__shfl_xor((int)bp, off);
            const double oba = __shfl_xor(ba, off);
            if (obp != 0xFFFFFFFFu && (bp == 0xFFFFFFFFu || oba < ba || (oba == ba && obp < bp))) {
                ba = oba;
                bp = obp;
            }
        }
        if (first == 0xFFFFFFFFu) break;  // nothing live left
        const uint32_t win = __builtin_isnan(first_a) ? first : bp;
        const uint32_t t = t0 + (win >> 4), li = (win >> 2) & 3u, lj = win & 3u, slot = lj * 4u + li;
        uint32_t live = 0;
        for (uint32_t w = 0; w < 4u; ++w) live += word_live(tile_word_load(tiles, (uint64_t)t * 4u + w));
        const uint32_t before = tile_len(flags[t] != 0, live);
        const uint32_t nsp = (live - 1u) <= sp ? 1u : 0u;
        if (lane == 0u) {
            uint32_t *wp = reinterpret_cast<uint32_t *>(tiles) + (uint64_t)t * 4u + (slot >> 2);
            const uint32_t v = __hip_atomic_load(wp, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(wp, v & ~(0xFFu << (8u * (slot & 3u))), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            flags[t] = (uint8_t)nsp;
            atomicAdd(ctr, 1ull);
        }
        __threadfence();
        used = used - before + tile_len(nsp != 0u, live - 1u);
    }
    if (used > alloc && lane == 0u) {
        // the write-back clamped to the whole tiles that fit
        uint64_t fit = 0;
        for (uint32_t t = t0; t < t1; ++t) {
            uint32_t live = 0;
            for (uint32_t w = 0; w < 4u; ++w) live += word_live(tile_word_load(tiles, (uint64_t)t * 4u + w));
            const uint32_t len = tile_len(flags[t] != 0, live);
            if (fit + len > alloc) break;
            fit += len;
        }
        atomicAdd(ctr + 1, 1ull);
        atomicAdd(ctr + 2, (unsigned long long)(used - fit));
    }
}

// The dense update's write-back (linear_disldo.hpp:1839-1880): one wave per
// block row, after its tiles were re-encoded by live count.
__global__ __launch_bounds__(256) void k_b4_merge(uint8_t *tiles, uint8_t *flags, const uint32_t *tile_start,
                                                  const uint32_t *tcol, const uint32_t *alloc, int64_t brows,
                                                  const float *is, const float *ois, int64_t n_in, int64_t n_out,
                                                  uint32_t sp, unsigned long long *ctr) {
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const int64_t br = (int64_t)blockIdx.x * WAVES_T + wave;
    if (br >= brows) return;
    const uint32_t t0 = tile_start[br], t1 = tile_start[br + 1];
    if (t0 == t1) return;
    uint64_t used = 0;
    for (uint32_t t = t0 + lane; t < t1; t += 64u) {
        const uint4 v = *reinterpret_cast<const uint4 *>(tiles + (uint64_t)t * 16u);
        used += tile_len(flags[t] != 0, word_live(v.x) + word_live(v.y) + word_live(v.z) + word_live(v.w));
    }
    for (int off = 32; off >= 1; off >>= 1) used += (uint64_t)__shfl_xor((long long)used, off);
    if (used <= alloc[br]) return;
    b4_merge_row_wave(tiles, flags, tcol, t0, t1, br, used, alloc[br], is, ois, n_in, n_out, sp, ctr);
}

// The sparse-gradient update of block4 tiles (sisldo_ops.hpp:848-1100).
struct SparseB4Args {
    const uint32_t *byte_start, *tile_start;
    const uint8_t *idx;
    uint8_t *tiles;
    int64_t brows, n_in, n_out, B, ntiles;
    const float *xT, *gT;      // gT as SparseTrainArgs
    float *dx;                 // [B][n_in], added into
    const float *vs, *os, *is, *ois;  // component 0 of the scales is read
    double *rowsum;            // [n_in][2], written for rows of block rows with tiles
    int rank;
    float lr, beta2, eps;
    int lr_per_row_nnz, damp;
    uint64_t seed;
    // the write-back after every (batch row, block row): tile_is_sparse,
    // the tiles' block columns, the rows' reserved tile bytes, switch_point
    // and the counters (b4_merge_row_wave)
    uint8_t *flags;
    const uint32_t *tcol, *alloc;
    uint32_t sp;
    unsigned long long *ctr;
};

// One wave per canonical block row; batch rows outermost, the row's tiles
// re-walked per batch row (4 tiles x 16 slots per pass, lanes (tile, li,
// lj)).  Each slot whose dy entry is nonzero steps its decoded weight and
// importance (no bounds) from the current byte and is re-quantized at once,
// stochastically in every layer class as the reference does, with draws
// splitmix64(seed + 2 id (+1)), id = (b * ntiles + t) * 16 + slot.  Lanes 0..3
// (one per tile row) add the slots' dx and fp64 row terms in (tile, lj)
// order per batch row, then into the row's sums, the reference's
// association.
__global__ __launch_bounds__(256) void k_sparse_train_b4(SparseB4Args a) {
    __shared__ uint32_t s_bc[WAVES_T][64];
    __shared__ float s_dx[WAVES_T][64];
    __shared__ double s_rg[WAVES_T][64], s_rgc[WAVES_T][64];
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const int64_t br = (int64_t)blockIdx.x * WAVES_T + wave;
    if (br >= a.brows) return;
    const uint32_t t0 = a.tile_start[br], t1 = a.tile_start[br + 1];
    if (t0 == t1) return;
    const int64_t B = a.B, rank = a.rank;
    const float nnz_row = (float)((t1 - t0) * 4u);
    const float eff_lr = a.lr_per_row_nnz ? a.lr / nnz_row : a.lr;
    const uint32_t tl = lane >> 4, li = (lane >> 2) & 3u, lj = lane & 3u;
    const int64_t row = br * 4 + li;
    const bool row_ok = row < a.n_in;
    const float val_scale = row_ok ? a.vs[row * rank] : 0.0f;
    const float imp_scale = (a.is && row_ok) ? a.is[row] : 1.0f;
    const int64_t my_row = br * 4 + lane;  // lanes 0..3: the row they sum
    double rs = 0.0, rsc = 0.0;
    const uint32_t end = a.byte_start[br + 1];
    const bool merge = a.lr != 0.0f && a.alloc != nullptr;
    for (int64_t b = 0; b < B; ++b) {
        const float in_val = row_ok ? a.xT[row * B + b] : 0.0f;
        float dxacc = 0.0f;
        double rgacc = 0.0, rgcacc = 0.0;
        uint64_t used = 0;  // the row's stored tile bytes after this batch row
        uint32_t pos = a.byte_start[br], carry = 0, ebase = t0;
        while (pos < end) {
            const Chunk ch = decode_chunk(a.idx, pos, end, carry);
            if (ch.T == 0ull) break;
            if (ch.term) s_bc[wave][ch.rank] = ch.col;
            wave_lds_sync();
            const uint32_t nt = (uint32_t)__popcll(ch.T);
            for (uint32_t sub = 0; sub < nt; sub += 4) {
                const uint32_t trank = sub + tl;
                const bool tile_ok = trank < nt;
                const uint32_t bc = tile_ok ? s_bc[wave][trank] : 0u;
                const int64_t t = (int64_t)ebase + trank;
                const int64_t col = (int64_t)bc * 4 + lj;
                const bool has = tile_ok && row_ok && col < a.n_out;
                const float dy_val = has ? a.gT[col * B + b] : 0.0f;
                const bool active = has && dy_val != 0.0f;
                float tdx = 0.0f;
                double rg = 0.0, rgc = 0.0;
                const uint32_t slot = lj * 4u + li;
                uint32_t newbyte = (merge && has) ? a.tiles[t * 16 + slot] : 0u;
                if (active) {
                    const uint32_t byte = a.tiles[t * 16 + slot];
                    const float w_decoded = fp4_decode(byte & 0xFu);
                    const float out_scale = a.os[col * rank];
                    const float combined_scale = val_scale * out_scale;
                    const float w = w_decoded * combined_scale;
                    tdx = w * dy_val;
                    if (a.lr != 0.0f) {
                        const float combined_imp_scale = imp_scale * (a.ois ? a.ois[col] : 1.0f);
                        const float grad = dy_val * in_val;
                        float imp = fp4_decode(byte >> 4) * combined_imp_scale;
                        const float contrib = in_val * w;
                        imp = a.beta2 * imp + (1.0f - a.beta2) * (grad * grad + contrib * contrib);
                        const float new_w = w + (a.damp ? (-eff_lr * grad) / (__builtin_sqrtf(imp) + a.eps)
                                                        : (-eff_lr * grad));
                        const uint64_t id = ((uint64_t)b * (uint64_t)a.ntiles + (uint64_t)t) * 16ull + slot;
                        const uint64_t base = a.seed + 2ull * id;
                        const uint32_t wq = fp4_encode_stochastic(new_w / combined_scale, splitmix64(base));
                        const uint32_t iq = fp4_encode_stochastic(imp / combined_imp_scale, splitmix64(base + 1ull));
                        a.tiles[t * 16 + slot] = (uint8_t)((iq << 4) | wq);
                        newbyte = (iq << 4) | wq;
                        rg = ((double)w_decoded * (double)out_scale) * (double)grad;
                        rgc = ((double)w_decoded * (double)out_scale) * (double)contrib;
                    }
                }
                const uint64_t act = __ballot(active);
                if (merge) {
                    // a rewritten tile is re-encoded by its live count
                    // (commit_dirty_tile_in_workspace); the row's stored
                    // bytes add up tile by tile
                    const uint64_t livem = __ballot(newbyte != 0u);
                    for (uint32_t u = 0; u < 4u && sub + u < nt; ++u) {
                        const uint32_t live = (uint32_t)__popcll((livem >> (16u * u)) & 0xFFFFull);
                        const bool dirty = ((act >> (16u * u)) & 0xFFFFull) != 0ull;
                        const int64_t tu = (int64_t)ebase + sub + u;
                        // lane 16u handles tile tu at every batch row: it
                        // alone reads and writes the tile's flag
                        uint32_t f = 0;
                        if (lane == 16u * u) {
                            f = dirty ? (live <= a.sp ? 1u : 0u) : (uint32_t)a.flags[tu];
                            if (dirty) a.flags[tu] = (uint8_t)f;
                        }
                        f = (uint32_t)__shfl((int)f, (int)(16u * u));
                        used += tile_len(f != 0u, live);
                    }
                }
                s_dx[wave][lane] = tdx;
                s_rg[wave][lane] = rg;
                s_rgc[wave][lane] = rgc;
                wave_lds_sync();
                if (lane < 4u) {
                    for (uint32_t u = 0; u < 4u && sub + u < nt; ++u) {
                        for (uint32_t j = 0; j < 4u; ++j) {
                            const uint32_t l = u * 16u + lane * 4u + j;
                            if (!((act >> l) & 1ull)) continue;
                            dxacc = dxacc + s_dx[wave][l];
                            rgacc = rgacc + s_rg[wave][l];
                            rgcacc = rgcacc + s_rgc[wave][l];
                        }
                    }
                }
                wave_lds_sync();
            }
            carry = chunk_advance(ch, pos, ebase);
        }
        if (lane < 4u && my_row < a.n_in) {
            a.dx[b * a.n_in + my_row] += dxacc;
            rs = rs + rgacc;
            rsc = rsc + rgcacc;
        }
        // the block row's workspace written back (sisldo_ops.hpp:1036-1052)
        if (merge && used > a.alloc[br]) {
            __threadfence();  // this batch row's tile writes, before the scan reads them
            b4_merge_row_wave(a.tiles, a.flags, a.tcol, t0, t1, br, used, a.alloc[br], a.is, a.ois, a.n_in,
                              a.n_out, a.sp, a.ctr);
        }
    }
    if (lane < 4u && my_row < a.n_in) {
        a.rowsum[2 * my_row] = rs;
        a.rowsum[2 * my_row + 1] = rsc;
    }
}

// The block rows' value-scale step of the sparse-gradient update
// (sisldo_ops.hpp:1068-1096): by the row index, step counter (row, 0), no
// finiteness guards.
__global__ __launch_bounds__(256) void k_sparse_train_vs_b4(const uint32_t *__restrict__ tile_start, int64_t n_in,
                                                            int rank, const double *__restrict__ rowsum, float *vs,
                                                            float *vs_imp, uint32_t *vs_step, float lr, float beta2,
                                                            float eps, const float *pow_tab) {
    const int64_t r = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (r >= n_in) return;
    const int64_t br = r >> 2;
    const uint32_t nt = tile_start[br + 1] - tile_start[br];
    if (nt == 0u) return;
    const double sum = rowsum[2 * r], sum_c = rowsum[2 * r + 1];
    if (sum == 0.0 && sum_c == 0.0) return;
    const float scale_eff_lr = lr / (float)(nt * 4u);
    const float g_agg = (float)sum, contrib_agg = (float)sum_c;
    const float new_vs_imp = beta2 * vs_imp[r] + (1.0f - beta2) * (g_agg * g_agg + contrib_agg * contrib_agg);
    const uint32_t step = vs_step[r * rank] + 1u;
    vs_step[r * rank] = step;
    const float bias_correction = 1.0f - pow_tab[step];
    const float hat = bias_correction > 0.0f ? new_vs_imp / bias_correction : new_vs_imp;
    vs_imp[r] = new_vs_imp;
    vs[r] = vs[r] - scale_eff_lr * g_agg / (__builtin_sqrtf(hat) + eps);
}

// dead_S[b*rank + k] = sum_col os_k(col) * dy[b][col] in fp64
// (linear_disldo.hpp:1995-2007): one block per (b, k).
__global__ __launch_bounds__(256) void k_dead_S(const float *__restrict__ os, const float *__restrict__ gT,
                                                int64_t n_out, int64_t B, int rank, double *__restrict__ dead_S) {
    __shared__ double part[256];
    const int64_t b = blockIdx.x / rank;
    const int k = (int)(blockIdx.x % rank);
    double s = 0.0;
    for (int64_t c = threadIdx.x; c < n_out; c += 256)
        s = s + (double)os[c * rank + k] * (double)gT[c * B + b];
    part[threadIdx.x] = s;
    __syncthreads();
    for (int h = 128; h > 0; h >>= 1) {
        if ((int)threadIdx.x < h) part[threadIdx.x] = part[threadIdx.x] + part[threadIdx.x + h];
        __syncthreads();
    }
    if (threadIdx.x == 0) dead_S[blockIdx.x] = part[0];
}

// Rows with no synapse: a two-moment step on value_scale
// (linear_disldo.hpp:2008-2040).
__global__ __launch_bounds__(256) void k_dead_rows(const uint32_t *__restrict__ elem_start,
                                                   const uint32_t *__restrict__ b4_tile_start, int64_t brows,
                                                   int64_t n_in, int64_t n_out, int64_t B, int rank,
                                                   const float *__restrict__ xT, const double *__restrict__ dead_S,
                                                   float *vs, float *vs_mom, float *vs_imp, float lr, float beta1,
                                                   float beta2, float eps) {
    const int64_t r = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (r >= n_in || elem_start[r + 1] != elem_start[r]) return;
    // a row in a block row holding tiles is not dead (linear_disldo.hpp:1986-1996)
    if (b4_tile_start && r / 4 < brows && b4_tile_start[r / 4 + 1] != b4_tile_start[r / 4]) return;
    for (int k = 0; k < rank; ++k) {
        double sum = 0.0;
        for (int64_t b = 0; b < B; ++b) {
            const float iv = xT[r * B + b];
            if (iv == 0.0f) continue;
            sum = sum + (double)iv * dead_S[b * rank + k];
        }
        if (sum == 0.0) continue;
        const float g = (float)sum;
        if (!finite_f(g)) continue;
        const int64_t i = r * rank + k;
        const float m = vs_mom[i], v = vs_imp[i];
        const float new_m = beta1 * m + (1.0f - beta1) * g;
        const float new_v = beta2 * v + (1.0f - beta2) * g * g;
        if (!finite_f(new_m) || !finite_f(new_v)) continue;
        const float dead_lr = lr / (float)n_out;
        const float new_vs = vs[i] - dead_lr * new_m / (__builtin_sqrtf(new_v) + eps);
        if (!finite_f(new_vs)) continue;
        vs_mom[i] = new_m;
        vs_imp[i] = new_v;
        vs[i] = new_vs;
    }
}

// output_scale's step (linear_disldo.hpp:2050-2080): one thread per column;
// its synapses' column-gradient terms are summed in shadow order (the
// column's synapses by ascending row, the reference's single-thread order).
// deg: out_degree as the reference's synaptogenesis policy keeps it, or NULL
// (then the column's stored synapses).
// b4: the block4 shadow (tile_start / idx per block column, tile ->
// canonical tile) and the tiles' terms, added after the scattered ones in
// (block row, tile row) order, or NULL.
struct B4ColTerms {
    const uint32_t *tile_start, *byte_start, *perm;
    const uint8_t *idx;
    const float *term;
    int64_t n_in;
};
__global__ __launch_bounds__(256) void k_train_cols(const uint32_t *__restrict__ t_elem_start,
                                                    const uint32_t *__restrict__ perm, int64_t n_out, int rank,
                                                    const float *__restrict__ mterm, float *os, float *os_imp,
                                                    uint32_t *os_step, float lr, float beta2, float eps,
                                                    const float *pow_tab, const int32_t *__restrict__ out_deg,
                                                    B4ColTerms b4) {
    const int64_t c = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (c >= n_out) return;
    const uint32_t s0 = t_elem_start[c], s1 = t_elem_start[c + 1];
    const int64_t deg = out_deg ? (int64_t)out_deg[c] : (int64_t)(s1 - s0);
    if (deg == 0) return;
    const float col_eff_lr = lr / (float)deg;
    for (int k = 0; k < rank; ++k) {
        float m = 0.0f, mc = 0.0f;
        for (uint32_t s = s0; s < s1; ++s) {
            const int64_t e = perm[s];
            m = m + mterm[e * 2 * rank + k];
            mc = mc + mterm[e * 2 * rank + rank + k];
        }
        if (b4.term) {
            const int64_t bcol = c >> 2;
            const uint32_t lj = (uint32_t)(c & 3);
            size_t pos = b4.byte_start[bcol];
            uint32_t brow = 0;
            for (uint32_t st = b4.tile_start[bcol]; st < b4.tile_start[bcol + 1]; ++st) {
                uint32_t v = 0;
                for (uint32_t sh = 0;; sh += 7) {
                    const uint8_t byte = b4.idx[pos++];
                    v |= (uint32_t)(byte & 0x7Fu) << sh;
                    if (!(byte & 0x80u)) break;
                }
                brow += v;
                const int64_t t = b4.perm[st];
                for (uint32_t li = 0; li < 4u; ++li) {
                    if ((int64_t)brow * 4 + li >= b4.n_in) continue;
                    const int64_t q = (t * 16 + lj * 4 + li) * 2 * rank;
                    m = m + b4.term[q + k];
                    mc = mc + b4.term[q + rank + k];
                }
            }
        }
        const int64_t i = c * rank + k;
        float osv = os[i], st = os_imp[i];
        uint32_t step = os_step[i];
        rmsprop_scale_update(osv, st, (float)(0.0 + (double)m), col_eff_lr, beta2, eps, (float)(0.0 + (double)mc),
                             step, pow_tab);
        os[i] = osv;
        os_imp[i] = st;
        os_step[i] = step;
    }
}

__global__ void k_perm_bytes(const uint8_t *__restrict__ src, const uint32_t *__restrict__ perm, int64_t n,
                             uint8_t *__restrict__ dst) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i < n) dst[i] = src[perm[i]];
}

inline unsigned nblk(int64_t n) { return (unsigned)((n + TPB - 1) / TPB); }

template <int RANK>
void launch_rows_rank(bool deferred, bool cols, dim3 grid, dim3 block, uint32_t lds, hipStream_t st,
                      const TrainArgs &a) {
    if (deferred) {
        if (cols) launch(k_train_rows<RANK, true, true>, grid, block, lds, st, a);
        else launch(k_train_rows<RANK, true, false>, grid, block, lds, st, a);
    } else {
        if (cols) launch(k_train_rows<RANK, false, true>, grid, block, lds, st, a);
        else launch(k_train_rows<RANK, false, false>, grid, block, lds, st, a);
    }
}

void launch_rows_kernel(int rank, bool deferred, bool cols, dim3 grid, dim3 block, uint32_t lds, hipStream_t st,
                        const TrainArgs &a) {
    switch (rank) {
        case 1: launch_rows_rank<1>(deferred, cols, grid, block, lds, st, a); break;
        case 2: launch_rows_rank<2>(deferred, cols, grid, block, lds, st, a); break;
        case 3: launch_rows_rank<3>(deferred, cols, grid, block, lds, st, a); break;
        default: launch_rows_rank<4>(deferred, cols, grid, block, lds, st, a); break;
    }
}

}  // namespace

void launch_train_rows(Layer &L, const float *xT, const float *gT, int64_t B, float *dx, const TrainParams &p,
                       uint64_t seed, hipStream_t st) {
    TrainArgs a{};
    a.byte_start = L.W.byte_start.p;
    a.elem_start = L.W.elem_start.p;
    a.idx = L.W.idx.p;
    a.val = L.W.val.p;
    a.n_in = L.n_in;
    a.n_out = L.n_out;
    a.B = B;
    a.xT = xT;
    a.gT = gT;
    a.dx = dx;
    a.vs = L.vs.p;
    a.vs_imp = L.vs_imp.p;
    a.vs_step = L.vs_step.p;
    a.os = L.os.p;
    a.is = L.is.p;
    a.ois = L.ois.p;
    a.pow_tab = L.pow_tab.p;
    a.mterm = L.output_scale_trainable ? L.mterm.p : nullptr;
    a.deferred = L.update_variant == UPDATE_RESYNC ? 1 : 0;
    a.no_scale = L.update_variant == UPDATE_NOSCALE ? 1 : 0;
    a.vs_read = L.vs.p;
    if (a.deferred) {
        L.def_w.ensure((size_t)std::max<int64_t>(1, L.W.nnz));
        L.def_i.ensure((size_t)std::max<int64_t>(1, L.W.nnz));
        a.def_w = L.def_w.p;
        a.def_i = L.def_i.p;
        if (L.rank > 1) {
            // rows write scale slots that other rows read: rows read a snapshot
            L.vs_snap.ensure((size_t)(L.n_in * L.rank));
            SILI_HIP(hipMemcpyAsync(L.vs_snap.p, L.vs.p, (size_t)(L.n_in * L.rank) * 4, hipMemcpyDeviceToDevice, st));
            a.vs_read = L.vs_snap.p;
        }
    }
    a.lr = p.lr;
    a.beta2 = p.beta2;
    a.eps = p.eps;
    a.min_decay_frac = p.min_decay_frac;
    a.max_abs_delta = p.max_abs_delta;
    a.max_ci = p.max_ci;
    a.zero_escape_eps = p.zero_escape_eps;
    a.lr_per_row_nnz = p.lr_per_row_nnz;
    a.damp = p.damp_by_importance;
    a.stochastic = L.stochastic_rounding ? 1 : 0;
    a.seed = seed;
    const dim3 grid((unsigned)((L.n_in + WAVES_T - 1) / WAVES_T)), block(256);
    const uint32_t lds = (uint32_t)(WAVES_T * (2 * B + 512) * sizeof(float));
    ProfScope ps("train_rows", st);
    launch_rows_kernel(L.rank, a.deferred != 0, a.mterm != nullptr, grid, block, lds, st, a);
    SILI_HIP(hipGetLastError());
}

void launch_sparse_train(Layer &L, const float *xT, const float *gT, int64_t B, float *dx, const TrainParams &p,
                         hipStream_t st) {
    L.train_rowsum.ensure((size_t)(2 * L.n_in));
    SparseTrainArgs a{};
    a.byte_start = L.W.byte_start.p;
    a.elem_start = L.W.elem_start.p;
    a.idx = L.W.idx.p;
    a.val = L.W.val.p;
    a.n_in = L.n_in;
    a.B = B;
    a.xT = xT;
    a.gT = gT;
    a.dx = dx;
    a.vs = L.vs.p;
    a.os = L.os.p;
    a.is = L.is.p;
    a.ois = L.ois.p;
    a.rowsum = L.train_rowsum.p;
    a.rank = L.rank;
    a.lr = p.lr;
    a.beta2 = p.beta2;
    a.eps = p.eps;
    a.lr_per_row_nnz = p.lr_per_row_nnz;
    a.damp = p.damp_by_importance;
    ProfScope ps("sparse_train_rows", st);
    launch(k_sparse_train_rows, dim3((unsigned)((L.n_in + WAVES_T - 1) / WAVES_T)), dim3(256),
           (uint32_t)(WAVES_T * (2 * B + 512) * sizeof(float)), st, a);
    launch(k_sparse_train_vs, dim3(nblk(L.n_in)), dim3(TPB), 0, st, (const uint32_t *)L.W.elem_start.p, L.n_in,
           L.rank, (const double *)L.train_rowsum.p, L.vs.p, L.vs_imp.p, L.vs_step.p, p.lr, p.beta2, p.eps,
           (const float *)L.pow_tab.p);
    SILI_HIP(hipGetLastError());
}

void launch_b4_merge(Layer &L, hipStream_t st) {
    if (L.B4.ntiles == 0) return;
    const uint32_t *tcol = b4_tile_cols(L);
    const uint32_t *alloc = b4res_device_alloc(L, st);
    unsigned long long *ctr = b4res_counters(L, st);
    ProfScope ps("b4_merge", st);
    launch(k_b4_merge, dim3((unsigned)((L.B4.brows + WAVES_T - 1) / WAVES_T)), dim3(256), 0, st, L.B4.tiles.p,
           L.B4.sparse.p, (const uint32_t *)L.B4.tile_start.p, tcol, alloc, L.B4.brows, (const float *)L.is.p,
           (const float *)L.ois.p, L.n_in, L.n_out, L.switch_point, ctr);
    SILI_HIP(hipGetLastError());
}

void launch_sparse_train_b4(Layer &L, const float *xT, const float *gT, int64_t B, float *dx,
                            const TrainParams &p, uint64_t seed, hipStream_t st) {
    if (L.B4.ntiles == 0) return;
    L.train_rowsum.ensure((size_t)(2 * L.n_in));
    SparseB4Args a{};
    a.byte_start = L.B4.byte_start.p;
    a.tile_start = L.B4.tile_start.p;
    a.idx = L.B4.idx.p;
    a.tiles = L.B4.tiles.p;
    a.brows = L.B4.brows;
    a.n_in = L.n_in;
    a.n_out = L.n_out;
    a.B = B;
    a.ntiles = L.B4.ntiles;
    a.xT = xT;
    a.gT = gT;
    a.dx = dx;
    a.vs = L.vs.p;
    a.os = L.os.p;
    a.is = L.is.p;
    a.ois = L.ois.p;
    a.rowsum = L.train_rowsum.p;
    a.rank = L.rank;
    a.lr = p.lr;
    a.beta2 = p.beta2;
    a.eps = p.eps;
    a.lr_per_row_nnz = p.lr_per_row_nnz;
    a.damp = p.damp_by_importance;
    a.seed = seed;
    a.flags = L.B4.sparse.p;
    a.tcol = b4_tile_cols(L);
    a.alloc = b4res_device_alloc(L, st);
    a.sp = L.switch_point;
    a.ctr = b4res_counters(L, st);
    ProfScope ps("sparse_train_b4", st);
    launch(k_sparse_train_b4, dim3((unsigned)((L.B4.brows + WAVES_T - 1) / WAVES_T)), dim3(256), 0, st, a);
    launch(k_sparse_train_vs_b4, dim3(nblk(L.n_in)), dim3(TPB), 0, st, (const uint32_t *)L.B4.tile_start.p, L.n_in,
           L.rank, (const double *)L.train_rowsum.p, L.vs.p, L.vs_imp.p, L.vs_step.p, p.lr, p.beta2, p.eps,
           (const float *)L.pow_tab.p);
    SILI_HIP(hipGetLastError());
}

void launch_train_b4(Layer &L, const float *xT, const float *gT, int64_t B, float *dx, const TrainParams &p,
                     uint64_t seed, hipStream_t st) {
    if (L.B4.ntiles == 0) return;
    B4TrainArgs a{};
    a.byte_start = L.B4.byte_start.p;
    a.tile_start = L.B4.tile_start.p;
    a.idx = L.B4.idx.p;
    a.tiles = L.B4.tiles.p;
    a.brows = L.B4.brows;
    a.n_in = L.n_in;
    a.n_out = L.n_out;
    a.B = B;
    a.nnz_scattered = L.W.nnz;
    a.xT = xT;
    a.gT = gT;
    a.dx = dx;
    a.vs = L.vs.p;
    a.vs_imp = L.vs_imp.p;
    a.vs_step = L.vs_step.p;
    a.os = L.os.p;
    a.is = L.is.p;
    a.ois = L.ois.p;
    a.pow_tab = L.pow_tab.p;
    if (L.output_scale_trainable) {
        L.b4term.ensure((size_t)(L.B4.ntiles * 16 * 2 * L.rank));
        a.b4term = L.b4term.p;
    }
    a.lr = p.lr;
    a.beta2 = p.beta2;
    a.eps = p.eps;
    a.min_decay_frac = p.min_decay_frac;
    a.max_abs_delta = p.max_abs_delta;
    a.max_ci = p.max_ci;
    a.zero_escape_eps = p.zero_escape_eps;
    a.lr_per_row_nnz = p.lr_per_row_nnz;
    a.damp = p.damp_by_importance;
    a.stochastic = L.stochastic_rounding ? 1 : 0;
    a.seed = seed;
    const dim3 grid((unsigned)((L.B4.brows + WAVES_B4 - 1) / WAVES_B4)), block(64 * WAVES_B4);
    const uint32_t shmem = (uint32_t)(WAVES_B4 * 4 * B * sizeof(float));  // B <= 1024: <= 32 KiB
    ProfScope ps("train_b4", st);
    switch (L.rank) {
        case 1: launch(k_train_b4<1>, grid, block, shmem, st, a); break;
        case 2: launch(k_train_b4<2>, grid, block, shmem, st, a); break;
        case 3: launch(k_train_b4<3>, grid, block, shmem, st, a); break;
        default: launch(k_train_b4<4>, grid, block, shmem, st, a); break;
    }
    SILI_HIP(hipGetLastError());
}

void launch_train_store(Layer &L, uint64_t seed, hipStream_t st) {
    if (L.update_variant != UPDATE_RESYNC || L.W.nnz == 0) return;
    TrainArgs a{};
    a.byte_start = L.W.byte_start.p;
    a.elem_start = L.W.elem_start.p;
    a.idx = L.W.idx.p;
    a.val = L.W.val.p;
    a.n_in = L.n_in;
    a.n_out = L.n_out;
    a.vs = L.vs.p;
    a.os = L.os.p;
    a.is = L.is.p;
    a.ois = L.ois.p;
    a.def_w = L.def_w.p;
    a.def_i = L.def_i.p;
    a.stochastic = L.stochastic_rounding ? 1 : 0;
    a.seed = seed;
    const dim3 grid((unsigned)((L.n_in + WAVES_T - 1) / WAVES_T)), block(256);
    ProfScope ps("train_store", st);
    switch (L.rank) {
        case 1: launch(k_train_store<1>, grid, block, 0, st, a); break;
        case 2: launch(k_train_store<2>, grid, block, 0, st, a); break;
        case 3: launch(k_train_store<3>, grid, block, 0, st, a); break;
        default: launch(k_train_store<4>, grid, block, 0, st, a); break;
    }
    SILI_HIP(hipGetLastError());
}

void launch_train_dead_rows(Layer &L, const float *xT, const float *gT, int64_t B, const TrainParams &p,
                            hipStream_t st) {
    L.dead_S.ensure((size_t)(B * L.rank));
    ProfScope ps("train_dead", st);
    launch(k_dead_S, dim3((unsigned)(B * L.rank)), dim3(256), 0, st, (const float *)L.os.p, gT, L.n_out, B, L.rank,
           L.dead_S.p);
    launch(k_dead_rows, dim3(nblk(L.n_in)), dim3(TPB), 0, st, (const uint32_t *)L.W.elem_start.p,
           L.B4.ntiles > 0 ? (const uint32_t *)L.B4.tile_start.p : nullptr, L.B4.brows, L.n_in, L.n_out, B,
           L.rank, xT, (const double *)L.dead_S.p, L.vs.p, L.vs_mom.p, L.vs_imp.p, p.lr, p.beta1, p.beta2, p.eps);
    SILI_HIP(hipGetLastError());
}

void launch_train_cols(Layer &L, const TrainParams &p, hipStream_t st) {
    ProfScope ps("train_cols", st);
    launch(k_train_cols, dim3(nblk(L.n_out)), dim3(TPB), 0, st, (const uint32_t *)L.Wt.elem_start.p,
           (const uint32_t *)L.Wt_perm.p, L.n_out, L.rank, (const float *)L.mterm.p, L.os.p, L.os_imp.p, L.os_step.p,
           p.lr, p.beta2, p.eps, (const float *)L.pow_tab.p,
           L.out_deg_tracked ? (const int32_t *)L.out_deg.p : nullptr,
           L.B4.ntiles > 0 ? B4ColTerms{L.B4t.tile_start.p, L.B4t.byte_start.p, L.B4t_perm.p, L.B4t.idx.p,
                                        L.b4term.p, L.n_in}
                           : B4ColTerms{nullptr, nullptr, nullptr, nullptr, nullptr, L.n_in});
    SILI_HIP(hipGetLastError());
}

void launch_shadow_val_refresh(Layer &L, hipStream_t st) {
    if (L.Wt.nnz == 0) return;
    ProfScope ps("train_shadow", st);
    launch(k_perm_bytes, dim3(nblk(L.Wt.nnz)), dim3(TPB), 0, st, (const uint8_t *)L.W.val.p,
           (const uint32_t *)L.Wt_perm.p, L.Wt.nnz, L.Wt.val.p);
    SILI_HIP(hipGetLastError());
}

}  // namespace sili
