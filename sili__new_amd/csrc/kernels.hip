// kernels.hip -- gfx950 kernels of the FP4 delta-CSR layer's hot path.
//
//   k_gather     scattered store, out[b,row] = sum_e w_e * in[col_e, b]
//                (forward on the shadow store, grad-input on the canonical one)
//   k_gather_b4  block4 contribution of the same, 4 output rows per block row
//   k_sddmm      nnz-sampled grad-W over the scattered store
//   k_sddmm_b4   nnz-sampled grad-W over every block4 slot
//   k_transpose  [B,n] -> [n,B] activations, fused sum_b |x| accumulators
//   k_densify_tiles  CSR activations -> the whole dense feature-major array
//   k_decode*    device decode of a store (export / parity / rebuild)
//
// Work item = one SegDesc decoded by one wave64.  The wave walks the
// segment's ULEB128 bytes 64 at a time (decode_chunk: ballot of terminator
// bytes, 7-bit group assembly, wave prefix sum of the deltas), stages the
// window's entries (column, dequantised weight) in its LDS slice, then
// consumes them with the batch spread over lanes: G entry groups of 64/G
// batch lanes each (G = 64 at batch 1, G = 1 at batch >= 64, where each lane
// owns KB batch columns).
#include "wave.hpp"

#include <algorithm>
#include <cstdlib>

namespace sili {

namespace {

constexpr int WAVES = 4;  // waves per 256-thread block

struct GArgs {
    const SegDesc *seg;
    int64_t nseg;
    const uint8_t *idx;
    const uint8_t *val;
    ScaleView sc;
    const float *in;
    int64_t in_ld;
    float *out;
    int64_t out_ld;
    int64_t nb;
    uint32_t in_bytes;  // readable bytes from `in` (buffer range for the fast kernels)
    int accumulate;     // float4 kernels: add to out instead of storing (column-block passes)
    int xcd;            // float4 kernels: XCD-contiguous block order (xcd_block)
    // k_gather_v4: split rows combined in order by their last item (GatherPlan)
    const uint32_t *elem_start;
    uint32_t *split_cnt;
    float *part;
    // k_gather_v4 with short rows (sh_seg != nullptr): blocks [0, n_lgblk)
    // take the work items seg[0, nseg) a wave each, the blocks after them the
    // short rows sh_seg[0, n_sh), up to SHORT_R_MAX to a wave
    const SegDesc *sh_seg;
    int64_t n_sh;
    uint32_t n_lgblk;
};

// Per-wave FP4 code -> value table (dequant by lookup).
__device__ __forceinline__ void fp4_table_init(float *tab) {
    const uint32_t lane = lane_id();
    if (lane < 16u) tab[lane] = fp4_decode(lane);
}

template <int G, int KB, int SKIP>
__global__ __launch_bounds__(256) void k_gather(GArgs a) {
    __shared__ uint32_t s_col[WAVES][64];
    __shared__ float s_w[WAVES][64];
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    __shared__ SegStage s_stage[WAVES];
    const int64_t si = (int64_t)blockIdx.x * WAVES + wave;
    if (si >= a.nseg) return;
    const SegDesc sd = a.seg[si];
    constexpr uint32_t BL = 64u / G;
    const uint32_t g = lane / BL, bl = lane % BL;
    const uint32_t row = sd.row;
    float acc[KB];
#pragma unroll
    for (int k = 0; k < KB; ++k) acc[k] = 0.0f;
    const StagedSeg sg = stage_segment(s_stage[wave], a.idx, a.val, sd);
    uint32_t pos = 0, carry = sd.base_col, ebase = sd.elem_begin;
    const uint32_t end = sg.end;
    while (pos < end) {
        const Chunk ch = decode_chunk(sg.idx, pos, end, carry);
        if (ch.T == 0ull) break;  // malformed stream: never spin
        if (ch.term) {
            const uint32_t code = (uint32_t)sg.val[ebase + ch.rank - sd.elem_begin] >> 4;
            s_col[wave][ch.rank] = ch.col;
            s_w[wave][ch.rank] = fp4_decode(code) * scale_at(a.sc, row, ch.col);
        }
        wave_lds_sync();
        const uint32_t n = (uint32_t)__popcll(ch.T);
        // U entries per group in flight: all loads issued before the FMAs
        constexpr uint32_t U = KB >= 4 ? 4u : 8u;
        uint32_t j = 0;
        for (; j + G * U <= n; j += G * U) {
            uint32_t c[U];
            float w[U], x[U][KB];
#pragma unroll
            for (uint32_t u = 0; u < U; ++u) {
                c[u] = s_col[wave][j + u * G + g];
                w[u] = s_w[wave][j + u * G + g];
            }
#pragma unroll
            for (uint32_t u = 0; u < U; ++u) {
                const float *src = a.in + (int64_t)c[u] * a.in_ld;
#pragma unroll
                for (int k = 0; k < KB; ++k) {
                    const int64_t b = (int64_t)bl + (int64_t)BL * k;
                    x[u][k] = b < a.nb ? src[b] : 0.0f;
                }
            }
#pragma unroll
            for (uint32_t u = 0; u < U; ++u)
#pragma unroll
                for (int k = 0; k < KB; ++k)
                    if (!skip_x<SKIP>(x[u][k])) acc[k] = __builtin_fmaf(w[u], x[u][k], acc[k]);
        }
        for (; j < n; j += G) {
            const uint32_t e = j + g;
            if (e < n) {
                const uint32_t c = s_col[wave][e];
                const float w = s_w[wave][e];
                const float *src = a.in + (int64_t)c * a.in_ld;
#pragma unroll
                for (int k = 0; k < KB; ++k) {
                    const int64_t b = (int64_t)bl + (int64_t)BL * k;
                    if (b < a.nb) {
                        const float x = src[b];
                        if (!skip_x<SKIP>(x)) acc[k] = __builtin_fmaf(w, x, acc[k]);
                    }
                }
            }
        }
        wave_lds_sync();
        carry = chunk_advance(ch, pos, ebase);
    }
    if constexpr (G > 1) {
#pragma unroll
        for (uint32_t off = BL; off < 64u; off <<= 1) acc[0] += __shfl_xor(acc[0], (int)off, 64);
    }
    if (g == 0) {
#pragma unroll
        for (int k = 0; k < KB; ++k) {
            const int64_t b = (int64_t)bl + (int64_t)BL * k;
            if (b < a.nb) {
                float *o = a.out + b * a.out_ld + row;
                if (sd.split & SEG_SPLIT) atomicAdd(o, acc[k]);
                else *o = acc[k];
            }
        }
    }
}

// Batch 1: each terminator lane applies its own entry (buffer gather of
// in[col]); one wave reduction per segment, no entry staging.
template <int SKIP>
__global__ __launch_bounds__(256) void k_gather_b1(GArgs a) {
    __shared__ SegStage s_stage[WAVES];
    __shared__ float s_fp4[WAVES][16];
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const int64_t si = (int64_t)blockIdx.x * WAVES + wave;
    if (si >= a.nseg) return;
    const SegDesc sd = a.seg[si];
    const uint32_t row = sd.row;
    fp4_table_init(s_fp4[wave]);
    const StagedSeg sg = stage_segment(s_stage[wave], a.idx, a.val, sd);
    const __amdgpu_buffer_rsrc_t rin = buffer_rsrc(a.in, a.in_bytes);
    const uint32_t ld_bytes = (uint32_t)a.in_ld * 4u;
    float acc = 0.0f;
    uint32_t pos = 0, carry = sd.base_col, ebase = sd.elem_begin;
    const uint32_t end = sg.end;
    while (pos < end) {
        const Chunk ch = decode_chunk(sg.idx, pos, end, carry);
        if (ch.T == 0ull) break;
        if (ch.term) {
            const float x = buffer_load_f1(rin, ch.col * ld_bytes);
            const uint32_t code = (uint32_t)sg.val[ebase + ch.rank - sd.elem_begin] >> 4;
            const float w = s_fp4[wave][code] * scale_at(a.sc, row, ch.col);
            if (!skip_x<SKIP>(x)) acc = __builtin_fmaf(w, x, acc);
        }
        carry = chunk_advance(ch, pos, ebase);
    }
    acc = group_sum_last<64>(acc);
    if (lane == 63u) {
        float *o = a.out + row;
        if (sd.split & SEG_SPLIT) atomicAdd(o, acc);
        else *o = acc;
    }
}

// Staged bytes of one segment for the batch-1 kernels, whose lane L owns
// the index bytes [8L, 8L+8): 64 lanes cover 512 bytes.
constexpr uint32_t B1_SEG_BYTES = 512;  // one 8-byte slice per lane covers a segment
static_assert(SEG_BYTES_MAX <= B1_SEG_BYTES, "one 8-byte slice per lane");
struct B1Stage {
    uint32_t idx[B1_SEG_BYTES / 4 + 8];  // idx[0] = 0, raw dwords from idx[1]
    uint32_t val[B1_SEG_BYTES / 4 + 8];
};

// Batch 1 with lane-parallel decode: lane L owns the index bytes
// [8L, 8L+8) of the segment (64 x 8 bytes cover SEG_BYTES_MAX) and decodes the
// varints whose last byte lies there (looking back over at most 4
// continuation bytes for a varint that starts in the previous slice).  Two
// wave scans give each lane its first entry index and the column before
// its slice; the lane then gathers in[col] for its (at most 8) entries with
// all loads in flight.  One wave reduction per segment.  The index bytes are
// staged realigned (segment byte p at LDS byte 4 + p, a zero dword in
// front: zero bytes end a lookback), so a lane's 12-byte window is three
// aligned dwords.  RANK1: scale rank 1 (row factor uniform per segment).
template <int SKIP, bool RANK1>
__global__ __launch_bounds__(256) void k_gather_b1s(GArgs a, uint32_t ent_bytes) {
    __shared__ B1Stage s_stage[WAVES];
    __shared__ float s_fp4[WAVES][16];
    __shared__ uint2 s_ent[WAVES][SEG_BYTES_MAX];
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const int64_t si = (int64_t)blockIdx.x * WAVES + wave;
    if (si >= a.nseg) return;
    const SegDesc sd = a.seg[si];
    fp4_table_init(s_fp4[wave]);
    B1Stage &S = s_stage[wave];
    const uint32_t end = sd.byte_end - sd.byte_begin < SEG_BYTES_MAX ? sd.byte_end - sd.byte_begin : SEG_BYTES_MAX;
    {
        // realigned copy: dst dword k (k >= 1) = segment bytes 4(k-1) .. 4(k-1)+3
        const uint32_t sh = sd.byte_begin & 3u;
        const uint32_t *src = reinterpret_cast<const uint32_t *>(a.idx + (sd.byte_begin & ~3u));
        const uint32_t nw = (end + 3u) / 4u + 1u;  // dwords 0 .. nw-1 written (<= 129)
        for (uint32_t k = lane; k < nw + 2u; k += 64u) {
            uint32_t d = 0;
            if (k >= 1u && k < nw) {
                const uint32_t lo = src[k - 1u], hi = src[k];
                d = sh ? __builtin_amdgcn_alignbyte(hi, lo, sh) : lo;
            }
            S.idx[k] = d;
        }
    }
    uint32_t voff = 0;  // value byte e of the segment is S.val byte voff + e
    stage_words(S.val, a.val, sd.elem_begin, sd.elem_end, voff);
    wave_lds_sync();
    const uint8_t *vals = reinterpret_cast<const uint8_t *>(S.val) + voff;
    const __amdgpu_buffer_rsrc_t rin = buffer_rsrc(a.in, a.in_bytes);
    const uint32_t ld_bytes = (uint32_t)a.in_ld * 4u;
    const uint32_t p0 = lane * 8u;
    // bytes [p0 - 4, p0 + 8): dwords 2L, 2L+1, 2L+2 of the realigned copy
    const uint32_t w0 = S.idx[2u * lane], w1 = S.idx[2u * lane + 1u], w2 = S.idx[2u * lane + 2u];
    uint32_t byte[12];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        byte[i] = (w0 >> (8 * i)) & 0xFFu;
        byte[4 + i] = (w1 >> (8 * i)) & 0xFFu;
        byte[8 + i] = (w2 >> (8 * i)) & 0xFFu;
    }
    // continuation prefix of the first varint ending in the slice
    uint32_t k = 0;
#pragma unroll
    for (int i = 3; i >= 0; --i) {
        const bool cont = (byte[i] & 0x80u) != 0u;
        k = (k == 3u - (uint32_t)i && cont) ? k + 1u : k;
    }
    uint32_t acc = 0, shift = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const bool use = (uint32_t)i >= 4u - k;
        acc = use ? (acc | ((byte[i] & 0x7Fu) << shift)) : acc;
        shift = use ? shift + 7u : shift;
    }
    uint32_t v[8];
    uint32_t cnt = 0, dsum = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint32_t b = byte[4 + i];
        const bool in_seg = p0 + (uint32_t)i < end;
        acc |= (b & 0x7Fu) << (shift < 32u ? shift : 0u);
        const bool term = in_seg && (b & 0x80u) == 0u;
        v[i] = term ? acc : 0xFFFFFFFFu;  // 0xFFFFFFFF: no entry ends here
        dsum += term ? acc : 0u;
        cnt += term ? 1u : 0u;
        acc = term ? 0u : acc;
        shift = term ? 0u : shift + 7u;
    }
    const uint32_t ebase = wave_incl_scan(cnt) - cnt;             // entries before this slice
    uint32_t col = sd.base_col + (wave_incl_scan(dsum) - dsum);   // column before this slice
    // entry table in LDS, segment order: (column, weight code)
    uint2 *ent = s_ent[wave];
    uint32_t e = ebase;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const bool has = v[i] != 0xFFFFFFFFu;
        col += has ? v[i] : 0u;
        if (has) ent[e] = make_uint2(col, (uint32_t)vals[e] >> 4);
        e += has ? 1u : 0u;
    }
    const uint32_t n = (uint32_t)__builtin_amdgcn_readlane((int)(ebase + cnt), 63);
    wave_lds_sync();
    // gather with 64 consecutive entries per load instruction, U in flight
    const float *tab = s_fp4[wave];
    const float rs = (RANK1 && a.sc.row) ? a.sc.row[sd.row] : 1.0f;
    // column factors (a zero-sized range when there are none: reads give 0)
    const __amdgpu_buffer_rsrc_t rent = buffer_rsrc(a.sc.ent ? a.sc.ent : a.in, a.sc.ent ? ent_bytes : 0u);
    constexpr uint32_t U = 4;
    float sum = 0.0f;
    for (uint32_t j = 0; j < n; j += 64u * U) {
        uint2 en[U];
        float xs[U], cs[U];
#pragma unroll
        for (uint32_t u = 0; u < U; ++u) {
            const uint32_t idx = j + u * 64u + lane;
            en[u] = idx < n ? ent[idx] : make_uint2(0xFFFFFFFFu, 0u);
            const bool ok = en[u].x != 0xFFFFFFFFu;
            xs[u] = buffer_load_f1(rin, ok ? en[u].x * ld_bytes : OOB_OFFSET);
            if constexpr (RANK1) cs[u] = a.sc.ent ? buffer_load_f1(rent, ok ? en[u].x * 4u : OOB_OFFSET) : 1.0f;
        }
#pragma unroll
        for (uint32_t u = 0; u < U; ++u) {
            if (en[u].x == 0xFFFFFFFFu) continue;
            float S;
            if constexpr (RANK1) S = a.sc.ent ? rs * cs[u] : rs;
            else S = scale_at(a.sc, sd.row, en[u].x);
            const float w = tab[en[u].y] * S;
            if (!skip_x<SKIP>(xs[u])) sum = __builtin_fmaf(w, xs[u], sum);
        }
    }
    sum = group_sum_last<64>(sum);
    if (lane == 63u) {
        float *o = a.out + sd.row;
        if (sd.split & SEG_SPLIT) atomicAdd(o, sum);
        else *o = sum;
    }
}

// Batch 1, persistent and software-pipelined: each wave walks segments
// s = w, w + W, w + 2W, ... (W = waves in the grid).  While it decodes and
// gathers segment s from LDS, the raw index / value dwords of segment s+W
// are already in flight into registers (3 + 3 per lane) and the descriptor
// of s+2W is loading, so the HBM latency of the weight stream hides behind
// the work of the previous segment.  Per segment: lane-parallel decode of
// 8-byte slices (as k_gather_b1s; the 12-byte window is read from the raw
// staged bytes with the segment's byte alignment, a zero dword in front),
// an LDS entry table in segment order, then the gather with 64 consecutive
// entries per load instruction and one wave reduction.


// XLDS (rank 1, no skip rules, in_ld == 1): the block first copies the
// whole input, times the column scale, into LDS (dynamic shared memory,
// n = a.in_bytes / 4 floats); the per-synapse gather then reads LDS and the
// weight is dec(code) * row scale (the column factor rides on x).
template <int SKIP, bool RANK1, bool XLDS = false>
__global__ __launch_bounds__(256) void k_gather_b1p(GArgs a, uint32_t ent_bytes) {
    __shared__ B1Stage s_stage[WAVES];
    __shared__ float s_fp4[WAVES][16];
    __shared__ uint32_t s_ent[WAVES][SEG_BYTES_MAX];  // col | code << 28
    extern __shared__ float s_x[];
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const int64_t W = (int64_t)gridDim.x * WAVES;
    if constexpr (XLDS) {
        const uint32_t nx = a.in_bytes / 4u;
        for (uint32_t i = threadIdx.x; i < nx; i += blockDim.x)
            s_x[i] = a.sc.ent ? a.in[i] * a.sc.ent[i] : a.in[i];
        __syncthreads();
    }
    int64_t si = (int64_t)blockIdx.x * WAVES + wave;
    if (si >= a.nseg) return;
    fp4_table_init(s_fp4[wave]);
    B1Stage &S = s_stage[wave];
    uint32_t *ent = s_ent[wave];
    const float *tab = s_fp4[wave];
    const __amdgpu_buffer_rsrc_t rin = buffer_rsrc(a.in, a.in_bytes);
    const __amdgpu_buffer_rsrc_t rent = buffer_rsrc(a.sc.ent ? a.sc.ent : a.in, a.sc.ent ? ent_bytes : 0u);
    const uint32_t ld_bytes = (uint32_t)a.in_ld * 4u;
    // raw dwords of a segment's index / value ranges (3 per lane each)
    auto load_data = [&](const SegDesc &d, uint32_t (&ri)[3], uint32_t (&rv)[3]) {
        const uint32_t *pi = reinterpret_cast<const uint32_t *>(a.idx + (d.byte_begin & ~3u));
        const uint32_t *pv = reinterpret_cast<const uint32_t *>(a.val + (d.elem_begin & ~3u));
        const uint32_t len = d.byte_end - d.byte_begin < SEG_BYTES_MAX ? d.byte_end - d.byte_begin : SEG_BYTES_MAX;
        const uint32_t ni = ((d.byte_begin & 3u) + len + 3u) >> 2;
        const uint32_t nv = ((d.elem_begin & 3u) + (d.elem_end - d.elem_begin) + 3u) >> 2;
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            const uint32_t q = lane + 64u * (uint32_t)k;
            ri[k] = q < ni ? pi[q] : 0u;
            rv[k] = q < nv ? pv[q] : 0u;
        }
    };
    SegDesc cur = a.seg[si];
    uint32_t ri[3], rv[3];
    load_data(cur, ri, rv);
    SegDesc nxt{};
    if (si + W < a.nseg) nxt = a.seg[si + W];
    for (; si < a.nseg; si += W) {
        // stage the current segment's bytes
        S.idx[0] = 0u;
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            const uint32_t q = lane + 64u * (uint32_t)k;
            if (q < SEG_BYTES_MAX / 4 + 7u) {
                S.idx[1u + q] = ri[k];
                S.val[q] = rv[k];
            }
        }
        // prefetch: data of the next segment, descriptor of the one after
        const bool more = si + W < a.nseg;
        SegDesc nn{};
        if (more) {
            load_data(nxt, ri, rv);
            if (si + 2 * W < a.nseg) nn = a.seg[si + 2 * W];
        }
        wave_lds_sync();
        const SegDesc &sd = cur;
        const uint32_t end = sd.byte_end - sd.byte_begin < SEG_BYTES_MAX ? sd.byte_end - sd.byte_begin : SEG_BYTES_MAX;
        const uint32_t ioff = sd.byte_begin & 3u;
        const uint8_t *vals = reinterpret_cast<const uint8_t *>(S.val) + (sd.elem_begin & 3u);
        const uint32_t p0 = lane * 8u;
        // bytes [p0 - 4, p0 + 8) = staged bytes [ioff + p0, ioff + p0 + 12)
        const uint32_t d0 = S.idx[2u * lane], d1 = S.idx[2u * lane + 1u], d2 = S.idx[2u * lane + 2u],
                       d3 = S.idx[2u * lane + 3u];
        const uint32_t w0 = ioff ? __builtin_amdgcn_alignbyte(d1, d0, ioff) : d0;
        const uint32_t w1 = ioff ? __builtin_amdgcn_alignbyte(d2, d1, ioff) : d1;
        const uint32_t w2 = ioff ? __builtin_amdgcn_alignbyte(d3, d2, ioff) : d2;
        uint32_t byte[12];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            byte[i] = lane ? (w0 >> (8 * i)) & 0xFFu : 0u;  // before the segment: terminators
            byte[4 + i] = (w1 >> (8 * i)) & 0xFFu;
            byte[8 + i] = (w2 >> (8 * i)) & 0xFFu;
        }
        uint32_t k = 0;
#pragma unroll
        for (int i = 3; i >= 0; --i) {
            const bool cont = (byte[i] & 0x80u) != 0u;
            k = (k == 3u - (uint32_t)i && cont) ? k + 1u : k;
        }
        uint32_t acc = 0, shift = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const bool use = (uint32_t)i >= 4u - k;
            acc = use ? (acc | ((byte[i] & 0x7Fu) << shift)) : acc;
            shift = use ? shift + 7u : shift;
        }
        uint32_t v[8];
        uint32_t cnt = 0, dsum = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t b = byte[4 + i];
            const bool in_seg = p0 + (uint32_t)i < end;
            acc |= (b & 0x7Fu) << (shift < 32u ? shift : 0u);
            const bool term = in_seg && (b & 0x80u) == 0u;
            v[i] = term ? acc : 0xFFFFFFFFu;
            dsum += term ? acc : 0u;
            cnt += term ? 1u : 0u;
            acc = term ? 0u : acc;
            shift = term ? 0u : shift + 7u;
        }
        const uint32_t ebase = wave_incl_scan(cnt) - cnt;
        uint32_t col = sd.base_col + (wave_incl_scan(dsum) - dsum);
        uint32_t e = ebase;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const bool has = v[i] != 0xFFFFFFFFu;
            col += has ? v[i] : 0u;
            if (has) ent[e] = col | (((uint32_t)vals[e] >> 4) << 28);
            e += has ? 1u : 0u;
        }
        const uint32_t n = (uint32_t)__builtin_amdgcn_readlane((int)(ebase + cnt), 63);
        wave_lds_sync();
        const float rs = (RANK1 && a.sc.row) ? a.sc.row[sd.row] : 1.0f;
        constexpr uint32_t U = 4;
        float sum = 0.0f;
        for (uint32_t j = 0; j < n; j += 64u * U) {
            uint32_t en[U];
            bool ok[U];
            float xs[U], cs[U];
#pragma unroll
            for (uint32_t u = 0; u < U; ++u) {
                const uint32_t idx = j + u * 64u + lane;
                ok[u] = idx < n;
                en[u] = ok[u] ? ent[idx] : 0u;
                const uint32_t c = en[u] & 0x0FFFFFFFu;
                if constexpr (XLDS) {
                    xs[u] = ok[u] ? s_x[c] : 0.0f;
                } else {
                    xs[u] = buffer_load_f1(rin, ok[u] ? c * ld_bytes : OOB_OFFSET);
                    if constexpr (RANK1) cs[u] = a.sc.ent ? buffer_load_f1(rent, ok[u] ? c * 4u : OOB_OFFSET) : 1.0f;
                }
            }
#pragma unroll
            for (uint32_t u = 0; u < U; ++u) {
                if (!ok[u]) continue;
                const uint32_t c = en[u] & 0x0FFFFFFFu;
                float Sv;
                if constexpr (XLDS) Sv = rs;
                else if constexpr (RANK1) Sv = a.sc.ent ? rs * cs[u] : rs;
                else Sv = scale_at(a.sc, sd.row, c);
                const float w = tab[en[u] >> 28] * Sv;
                if (!skip_x<SKIP>(xs[u])) sum = __builtin_fmaf(w, xs[u], sum);
            }
        }
        sum = group_sum_last<64>(sum);
        if (lane == 63u) {
            float *o = a.out + sd.row;
            if (sd.split & SEG_SPLIT) atomicAdd(o, sum);
            else *o = sum;
        }
        wave_lds_sync();  // LDS buffers are rewritten by the next iteration
        cur = nxt;
        nxt = nn;
    }
}

// Decode a whole staged segment into an LDS entry table: ent[k] = (byte
// offset of entry k's input row, weight bits), k < n; the table is padded up
// to a multiple of `step` with out-of-range offsets (their buffer loads read
// 0).  Returns n.  `ent` holds at least SEG_BYTES_MAX + 64 entries.
__device__ __forceinline__ uint32_t decode_segment_entries(const StagedSeg &sg, const SegDesc &sd,
                                                           const ScaleView &sc, const float *fp4tab,
                                                           uint32_t ld_bytes, uint32_t step, uint2 *ent) {
    const uint32_t lane = lane_id();
    uint32_t pos = 0, carry = sd.base_col, ebase = sd.elem_begin;
    while (pos < sg.end) {
        const Chunk ch = decode_chunk(sg.idx, pos, sg.end, carry);
        if (ch.T == 0ull) break;
        if (ch.term) {
            const uint32_t e = ebase - sd.elem_begin + ch.rank;
            const uint32_t code = (uint32_t)sg.val[e] >> 4;
            const float w = fp4tab[code] * scale_at(sc, sd.row, ch.col);
            ent[e] = make_uint2(ch.col * ld_bytes, __builtin_bit_cast(uint32_t, w));
        }
        carry = chunk_advance(ch, pos, ebase);
    }
    const uint32_t n = ebase - sd.elem_begin;
    const uint32_t npad = (n + step - 1u) / step * step;
    for (uint32_t k = n + lane; k < npad; k += 64u) ent[k] = make_uint2(OOB_OFFSET, 0u);
    wave_lds_sync();
    return n;
}

// float4 along the batch: groups of BL lanes take one entry each (G = 64/BL
// entries per load instruction); lane bl of a group owns float4 chunks
// q = bl + BL*k (k < KB) of the entry's feature-major input row.  The whole
// segment is decoded first (decode_segment_entries); the gather loop then
// keeps U loads per lane in flight with no predicates.  Needs nb % 4 == 0,
// in_ld % 4 == 0 and a 16-byte aligned `in`.
constexpr uint32_t ENT_CAP = SEG_BYTES_MAX + 64u;

// Block epilogue of the float4 kernels: out[b, row] for the block's (up to
// WAVES) segments.  Each wave leaves its nb results in its own LDS slice
// (`slice`, >= nb floats; lanes of group 0 hold float4 chunk q = bl + BL*k),
// then the block writes them with consecutive lanes on consecutive rows, so
// consecutive segments (rows) of one batch index leave as one run instead
// of WAVES scattered 4-byte stores.  Split rows add atomically, or are
// combined in order (below).  Every thread of the block must call this (it
// holds a block barrier).
// Split rows, without float atomics (sc.part != nullptr): a wave holding one
// work item of a split row leaves its partial sums in part[si * nb ...]; the
// last item of the row to finish (its entries counted into cnt[row] against
// the row's entries) adds the row's items in item order and writes the row,
// then clears the counter.  The result does not depend on the finishing order.
// The partials cross compute units and XCDs (whose L2s are not coherent with
// each other), so they move as agent-scope atomic stores and loads (written
// through to, and read from, the agent's coherence point); the wave waits for
// its stores to complete before it counts its arrival.  A device-scope fence
// would order them too, but it writes back and invalidates the whole L2 of
// the XCD, which the gather's input reuse depends on.
struct SplitCombine {
    const SegDesc *seg;
    int64_t nseg;
    const uint32_t *elem_start;
    uint32_t *cnt;
    float *part;  // nullptr: split rows add with atomics
};

// s_waitcnt vmcnt(0) (gfx9 encoding: expcnt and lgkmcnt left at their maxima)
constexpr int WAITCNT_VM0 = 0x0F70;

template <int BL, int KB>
__device__ __forceinline__ void store_rows_block(const float4 (&acc)[KB], bool active, uint32_t row,
                                                 bool split, uint32_t nq, float *slice_base,
                                                 uint32_t slice_stride, float *out, int64_t out_ld,
                                                 bool accumulate = false,
                                                 SplitCombine sc = SplitCombine{nullptr, 0, nullptr, nullptr, nullptr},
                                                 int64_t si = 0, uint32_t n_items = 0) {
    __shared__ uint32_t s_row[WAVES];
    __shared__ uint32_t s_flag[WAVES];  // bit 0: active, bit 1: split (atomics), bit 2: split (combined)
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const uint32_t g = lane / BL, bl = lane % BL;
    float *slice = slice_base + wave * slice_stride;
    const bool combine = split && sc.part != nullptr;
    if (active && g == 0) {
#pragma unroll
        for (int k = 0; k < KB; ++k) {
            const uint32_t q = bl + BL * (uint32_t)k;
            if (q < nq) *reinterpret_cast<float4 *>(slice + q * 4u) = acc[k];
        }
    }
    if (lane == 0) {
        s_row[wave] = row;
        s_flag[wave] = (active ? 1u : 0u) | (split && !combine ? 2u : 0u) | (combine ? 4u : 0u);
    }
    __syncthreads();
    const uint32_t nb = nq * 4u;
    for (uint32_t i = threadIdx.x; i < nb * WAVES; i += blockDim.x) {
        const uint32_t w = i % WAVES, b = i / WAVES;
        const uint32_t f = s_flag[w];
        if (!(f & 1u) || (f & 4u)) continue;
        const float v = slice_base[w * slice_stride + b];
        float *o = out + (int64_t)b * out_ld + s_row[w];
        if (f & 2u) atomicAdd(o, v);
        else *o = accumulate ? *o + v : v;  // (a row with one work item: this wave alone writes it)
    }
    if (active && combine) {
        float *dst = sc.part + si * (int64_t)nb;
        for (uint32_t b = lane; b < nb; b += 64u)
            __hip_atomic_store(dst + b, slice[b], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");  // (keeps the stores above the wait)
        __builtin_amdgcn_s_waitcnt(WAITCNT_VM0);
        uint32_t last = 0;
        if (lane == 0) {
            const uint32_t old = __hip_atomic_fetch_add(sc.cnt + row, n_items, __ATOMIC_RELAXED,
                                                        __HIP_MEMORY_SCOPE_AGENT);
            last = (old + n_items == sc.elem_start[row + 1] - sc.elem_start[row]) ? 1u : 0u;
        }
        last = (uint32_t)__shfl((int)last, 0);
        if (last) {
            int64_t k0 = si, k1 = si + 1;
            while (k0 > 0 && sc.seg[k0 - 1].row == row) --k0;
            while (k1 < sc.nseg && sc.seg[k1].row == row) ++k1;
            for (uint32_t b = lane; b < nb; b += 64u) {
                float s = 0.0f;
                for (int64_t k = k0; k < k1; ++k)
                    s += __hip_atomic_load(sc.part + k * (int64_t)nb + b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                float *o = out + (int64_t)b * out_ld + row;
                *o = accumulate ? *o + s : s;
            }
            if (lane == 0) __hip_atomic_store(sc.cnt + row, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}



// Short rows, up to SHORT_R_MAX to a wave (the blocks of k_gather_v4 past
// a.n_lgblk): every item of a.sh_seg is a whole row of at most
// SHORT_ROW_BYTES index bytes, and wave gi of these blocks takes items
// [gi*R, gi*R + R), R = SHORT_R_MAX.  A wave per such row would spend its
// staging, decode and epilogue latency on a handful of entries; here
//   - the rows' index and value bytes are staged back to back (32 lanes per
//     row, byte loads, all issued before the first wait);
//   - 64-byte windows are decoded as in decode_chunk, the column scan
//     restarting at each row's first byte (a segmented scan over the head
//     flags); each entry's row is the last head at or before it (a running
//     maximum of the row ids), so the scales see the right row;
//   - lane group g (BL lanes, float4 batch chunks as in the segment path)
//     accumulates rows g, g + G, ... of the wave in registers;
//   - the results go through the wave's entry table to a block epilogue that
//     writes the block's rows per batch index (stores, or adds with
//     a.accumulate).
// The entry table holds at most SEG_BYTES_MAX entries while decoding; its
// tail (entries SEG_BYTES_MAX ..) holds the head flags.  Needs a.nb <=
// SHORT_MAX_BATCH (R * nb floats fit the table).
// The float4 gather shapes that hold the short-row path: batch chunks of at
// most SHORT_MAX_BATCH columns (larger shapes would carry its registers).
constexpr bool short_rows_shape(int BL, int KB) { return 4 * BL * KB <= (int)SHORT_MAX_BATCH; }

template <int BL, int KB, int SKIP>
__device__ __forceinline__ void gather_short_body(const GArgs &a, uint32_t sblk, SegStage *stage,
                                                  uint2 (*ents)[ENT_CAP], float (*fp4s)[16]) {
    constexpr uint32_t G = 64u / BL;
    constexpr uint32_t RPG = (SHORT_R_MAX + G - 1u) / G;  // rows per lane group
    constexpr uint32_t US = KB * RPG >= 4u ? 1u : 2u;     // entries per row in flight
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const uint32_t g = lane / BL, bl = lane % BL;
    const uint32_t nq = (uint32_t)(a.nb >> 2), nbv = nq * 4u;
    const int64_t i0 = ((int64_t)sblk * WAVES + wave) * SHORT_R_MAX;
    const uint32_t nrows = i0 < a.n_sh ? (uint32_t)min<int64_t>((int64_t)SHORT_R_MAX, a.n_sh - i0) : 0u;
    SegStage &S = stage[wave];
    uint2 *ent = ents[wave];
    uint32_t *rowid = S.idx;  // after the decode: the wave's rows, then their count
    if (nrows > 0) {
        fp4_table_init(fp4s[wave]);
        uint32_t nby = 0, nen = 0, row = 0, bb = 0, eb = 0;
        if (lane < nrows) {
            const SegDesc d = a.sh_seg[i0 + lane];
            nby = d.byte_end - d.byte_begin;
            nen = d.elem_end - d.elem_begin;
            row = d.row;
            bb = d.byte_begin;
            eb = d.elem_begin;
        }
        const uint32_t binc = wave_incl_scan(nby), einc = wave_incl_scan(nen);
        const uint32_t boff = binc - nby, eoff = einc - nen;
        const uint32_t tot_b = (uint32_t)__builtin_amdgcn_readlane((int)binc, 63);
        uint8_t *sidx = reinterpret_cast<uint8_t *>(S.idx);
        uint8_t *sval = reinterpret_cast<uint8_t *>(S.val);
        uint8_t *hd = reinterpret_cast<uint8_t *>(ent + SEG_BYTES_MAX);
        for (uint32_t i = lane; i < SEG_BYTES_MAX / 4u; i += 64u) reinterpret_cast<uint32_t *>(hd)[i] = 0u;
        // the rows' bytes, two rows per pass (32 lanes each)
        uint32_t bv[SHORT_R_MAX / 2], vv[SHORT_R_MAX / 2];
        const uint32_t npass = (nrows + 1u) >> 1;
#pragma unroll
        for (uint32_t p = 0; p < SHORT_R_MAX / 2; ++p) {
            const uint32_t ri = 2u * p + (lane >> 5), off = lane & 31u;
            const uint32_t rb = (uint32_t)__shfl((int)bb, (int)ri), rn = (uint32_t)__shfl((int)nby, (int)ri);
            const uint32_t re = (uint32_t)__shfl((int)eb, (int)ri), rm = (uint32_t)__shfl((int)nen, (int)ri);
            bv[p] = (p < npass && off < rn) ? (uint32_t)a.idx[rb + off] : 0u;
            vv[p] = (p < npass && off < rm) ? (uint32_t)a.val[re + off] : 0u;
        }
#pragma unroll
        for (uint32_t p = 0; p < SHORT_R_MAX / 2; ++p) {
            const uint32_t ri = 2u * p + (lane >> 5), off = lane & 31u;
            const uint32_t rn = (uint32_t)__shfl((int)nby, (int)ri), rm = (uint32_t)__shfl((int)nen, (int)ri);
            const uint32_t ro = (uint32_t)__shfl((int)boff, (int)ri), rv = (uint32_t)__shfl((int)eoff, (int)ri);
            if (p < npass && off < rn) sidx[ro + off] = (uint8_t)bv[p];
            if (p < npass && off < rm) sval[rv + off] = (uint8_t)vv[p];
        }
        if (lane < nrows && nby > 0u) hd[boff] = (uint8_t)(lane + 1u);  // row id + 1 at its first byte
        wave_lds_sync();
        // decode, the scans restarting at row starts
        const float *tab = fp4s[wave];
        const uint32_t ld_bytes = (uint32_t)a.in_ld * 4u;
        uint32_t pos = 0, carry = 0, crow = 0, ebase = 0;
        while (pos < tot_b) {
            const Chunk ch = decode_chunk(sidx, pos, tot_b, 0u);
            if (ch.T == 0ull) break;
            const uint32_t p = pos + lane;
            const uint32_t rid = p < tot_b ? (uint32_t)hd[p] : 0u;
            const uint64_t H = __ballot(rid != 0u);
            const uint64_t le = lane == 63u ? ~0ull : ((2ull << lane) - 1ull);
            const bool headed = (H & le) != 0ull;
            const uint32_t col = wave_seg_scan(ch.v, rid != 0u ? 1u : 0u) + (headed ? 0u : carry);
            const uint32_t mr = wave_max_scan(rid);
            const uint32_t rl = headed ? mr - 1u : crow;
            const uint32_t grow = (uint32_t)__shfl((int)row, (int)rl);
            if (ch.term) {
                const uint32_t e = ebase + ch.rank;
                const float w = tab[(uint32_t)sval[e] >> 4] * scale_at(a.sc, grow, col);
                ent[e] = make_uint2(col * ld_bytes, __builtin_bit_cast(uint32_t, w));
            }
            const uint32_t hi = 63u - (uint32_t)__clzll(ch.T);
            carry = uniform((uint32_t)__shfl((int)col, (int)hi));
            crow = uniform((uint32_t)__shfl((int)rl, (int)hi));
            pos += hi + 1u;
            ebase += (uint32_t)__popcll(ch.T);
        }
        wave_lds_sync();
        // each lane group's rows
        const __amdgpu_buffer_rsrc_t rin = buffer_rsrc(a.in, a.in_bytes);
        uint32_t lane_off[KB];
#pragma unroll
        for (int k = 0; k < KB; ++k) {
            const uint32_t q = bl + BL * (uint32_t)k;
            lane_off[k] = q < nq ? q * 16u : OOB_OFFSET;
        }
        uint32_t eo[RPG], ne[RPG], nmax = 0;
#pragma unroll
        for (uint32_t t = 0; t < RPG; ++t) {
            const uint32_t i = g + G * t;
            const uint32_t src = i < 64u ? i : 0u;
            eo[t] = (uint32_t)__shfl((int)eoff, (int)src);
            const uint32_t n = (uint32_t)__shfl((int)nen, (int)src);
            ne[t] = i < nrows ? n : 0u;
            nmax = max(nmax, ne[t]);
        }
        float4 acc[RPG][KB];
#pragma unroll
        for (uint32_t t = 0; t < RPG; ++t)
#pragma unroll
            for (int k = 0; k < KB; ++k) acc[t][k] = make_float4(0.f, 0.f, 0.f, 0.f);
        for (uint32_t j = 0; j < nmax; j += US) {
            uint2 e[RPG][US];
            float4 x[RPG][US][KB];
#pragma unroll
            for (uint32_t t = 0; t < RPG; ++t)
#pragma unroll
                for (uint32_t u = 0; u < US; ++u)
                    e[t][u] = j + u < ne[t] ? ent[eo[t] + j + u] : make_uint2(OOB_OFFSET, 0u);
#pragma unroll
            for (uint32_t t = 0; t < RPG; ++t)
#pragma unroll
                for (uint32_t u = 0; u < US; ++u)
#pragma unroll
                    for (int k = 0; k < KB; ++k) x[t][u][k] = buffer_load_f4(rin, e[t][u].x + lane_off[k]);
#pragma unroll
            for (uint32_t t = 0; t < RPG; ++t)
#pragma unroll
                for (uint32_t u = 0; u < US; ++u) {
                    const float w = __builtin_bit_cast(float, e[t][u].y);
#pragma unroll
                    for (int k = 0; k < KB; ++k) {
                        const float4 xv = x[t][u][k];
                        float4 &A = acc[t][k];
                        if constexpr (SKIP == SKIP_NONE) {
                            A.x = __builtin_fmaf(w, xv.x, A.x);
                            A.y = __builtin_fmaf(w, xv.y, A.y);
                            A.z = __builtin_fmaf(w, xv.z, A.z);
                            A.w = __builtin_fmaf(w, xv.w, A.w);
                        } else {
                            if (!skip_x<SKIP>(xv.x)) A.x = __builtin_fmaf(w, xv.x, A.x);
                            if (!skip_x<SKIP>(xv.y)) A.y = __builtin_fmaf(w, xv.y, A.y);
                            if (!skip_x<SKIP>(xv.z)) A.z = __builtin_fmaf(w, xv.z, A.z);
                            if (!skip_x<SKIP>(xv.w)) A.w = __builtin_fmaf(w, xv.w, A.w);
                        }
                    }
                }
        }
        wave_lds_sync();  // every group is done with the entry table: it becomes the result slice
        float *slice = reinterpret_cast<float *>(ent);
#pragma unroll
        for (uint32_t t = 0; t < RPG; ++t) {
            const uint32_t i = g + G * t;
            if (i < nrows) {
#pragma unroll
                for (int k = 0; k < KB; ++k) {
                    const uint32_t q = bl + BL * (uint32_t)k;
                    if (q < nq) *reinterpret_cast<float4 *>(slice + i * nbv + q * 4u) = acc[t][k];
                }
            }
        }
        if (lane < nrows) rowid[lane] = row;
    }
    if (lane == 0) rowid[SHORT_R_MAX] = nrows;
    __syncthreads();
    // the block's rows per batch index: consecutive threads on consecutive rows
    constexpr uint32_t PER_B = WAVES * SHORT_R_MAX;
    for (uint32_t i = threadIdx.x; i < nbv * PER_B; i += blockDim.x) {
        const uint32_t r = i % SHORT_R_MAX, w = (i / SHORT_R_MAX) % WAVES, b = i / PER_B;
        if (r >= stage[w].idx[SHORT_R_MAX]) continue;
        const float v = reinterpret_cast<const float *>(ents[w])[r * nbv + b];
        float *o = a.out + (int64_t)b * a.out_ld + stage[w].idx[r];
        *o = a.accumulate ? *o + v : v;
    }
}

template <int BL, int KB, int U, int SKIP>
__global__ __attribute__((amdgpu_flat_work_group_size(1, 256), amdgpu_waves_per_eu(KB <= 2 && U <= 4 ? 8 : 1)))
void k_gather_v4(GArgs a) {
    __shared__ SegStage s_stage[WAVES];
    __shared__ uint2 s_ent[WAVES][ENT_CAP];
    __shared__ float s_fp4[WAVES][16];
    constexpr uint32_t G = 64u / BL;
    constexpr uint32_t STEP = G * U;
    if constexpr (short_rows_shape(BL, KB)) {
        if (a.sh_seg != nullptr && blockIdx.x >= a.n_lgblk) {
            gather_short_body<BL, KB, SKIP>(a, blockIdx.x - a.n_lgblk, s_stage, s_ent, s_fp4);
            return;
        }
    }
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const uint32_t nlb = a.sh_seg != nullptr ? a.n_lgblk : gridDim.x;
    const uint32_t bid = a.xcd ? xcd_block(blockIdx.x, nlb) : blockIdx.x;
    const int64_t si = (int64_t)bid * WAVES + wave;
    const bool active = si < a.nseg;  // inactive waves still join the block epilogue
    const uint32_t g = lane / BL, bl = lane % BL;
    const uint32_t nq = (uint32_t)(a.nb >> 2);
    float4 acc[KB];
#pragma unroll
    for (int k = 0; k < KB; ++k) acc[k] = make_float4(0.f, 0.f, 0.f, 0.f);
    SegDesc sd{};
    if (active) {
    sd = a.seg[si];
    fp4_table_init(s_fp4[wave]);
    const StagedSeg sg = stage_segment(s_stage[wave], a.idx, a.val, sd);
    const __amdgpu_buffer_rsrc_t rin = buffer_rsrc(a.in, a.in_bytes);
    uint32_t lane_off[KB];
#pragma unroll
    for (int k = 0; k < KB; ++k) {
        const uint32_t q = bl + BL * (uint32_t)k;
        lane_off[k] = q < nq ? q * 16u : OOB_OFFSET;  // chunks past the batch read 0
    }
    uint2 *ent = s_ent[wave];
    const uint32_t n = decode_segment_entries(sg, sd, a.sc, s_fp4[wave], (uint32_t)a.in_ld * 4u, STEP, ent);
    for (uint32_t j = 0; j < n; j += STEP) {
        uint2 e[U];
        float4 x[U][KB];
#pragma unroll
        for (int u = 0; u < U; ++u) e[u] = ent[j + (uint32_t)u * G + g];
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int k = 0; k < KB; ++k) x[u][k] = buffer_load_f4(rin, e[u].x + lane_off[k]);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const float w = __builtin_bit_cast(float, e[u].y);
#pragma unroll
            for (int k = 0; k < KB; ++k) {
                if constexpr (SKIP == SKIP_NONE) {
                    acc[k].x = __builtin_fmaf(w, x[u][k].x, acc[k].x);
                    acc[k].y = __builtin_fmaf(w, x[u][k].y, acc[k].y);
                    acc[k].z = __builtin_fmaf(w, x[u][k].z, acc[k].z);
                    acc[k].w = __builtin_fmaf(w, x[u][k].w, acc[k].w);
                } else {
                    // padding reads x = 0 and is skipped like a zero input
                    if (!skip_x<SKIP>(x[u][k].x)) acc[k].x = __builtin_fmaf(w, x[u][k].x, acc[k].x);
                    if (!skip_x<SKIP>(x[u][k].y)) acc[k].y = __builtin_fmaf(w, x[u][k].y, acc[k].y);
                    if (!skip_x<SKIP>(x[u][k].z)) acc[k].z = __builtin_fmaf(w, x[u][k].z, acc[k].z);
                    if (!skip_x<SKIP>(x[u][k].w)) acc[k].w = __builtin_fmaf(w, x[u][k].w, acc[k].w);
                }
            }
        }
    }
    // combine the G entry groups (lanes bl, bl+BL, ...)
#pragma unroll
    for (uint32_t off = BL; off < 64u; off <<= 1)
#pragma unroll
        for (int k = 0; k < KB; ++k) {
            acc[k].x += __shfl_xor(acc[k].x, (int)off, 64);
            acc[k].y += __shfl_xor(acc[k].y, (int)off, 64);
            acc[k].z += __shfl_xor(acc[k].z, (int)off, 64);
            acc[k].w += __shfl_xor(acc[k].w, (int)off, 64);
        }
    wave_lds_sync();  // the entry table is reused as this wave's output slice
    }
    store_rows_block<BL, KB>(acc, active, sd.row, (sd.split & SEG_SPLIT) != 0, nq,
                             reinterpret_cast<float *>(&s_ent[0][0]), ENT_CAP * 2u, a.out, a.out_ld,
                             a.accumulate != 0, SplitCombine{a.seg, a.nseg, a.elem_start, a.split_cnt, a.part},
                             si, sd.elem_end - sd.elem_begin);
}

struct BArgs {
    const SegDesc *seg;
    int64_t nseg;
    const uint8_t *idx;
    const uint8_t *tiles;
    int64_t rows, cols;
    ScaleView sc;
    const float *in;
    int64_t in_ld;
    float *out;
    int64_t out_ld;
    int64_t nb;
    // k_gather_b4_v4 only: 0 for a (segments, batch chunks) grid; else the
    // segment blocks per batch chunk of a 1-D grid taken in XCD-contiguous
    // order chunk-major, so that each XCD works on one batch chunk (its L2
    // then holds only that chunk's share of every input row)
    uint32_t xq_gx;
};

// SKIP: SKIP_NONE (dense paths), SKIP_ZERO (entry value 0 skipped), or
// SKIP_POSZERO, which also skips dead (byte 0) slots -- the sparse-input
// forward only visits live slots of active rows (sisldo_ops.hpp:519-531).
template <int G, int KB, int SKIP>
__global__ __launch_bounds__(256) void k_gather_b4(BArgs a) {
    __shared__ uint32_t s_bc[WAVES][64];
    __shared__ uint32_t s_t[WAVES][64];
    __shared__ __align__(16) float s_w[WAVES][64 * 16];
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const int64_t si = (int64_t)blockIdx.x * WAVES + wave;
    if (si >= a.nseg) return;
    const SegDesc sd = a.seg[si];
    constexpr uint32_t BL = 64u / G;
    const uint32_t g = lane / BL, bl = lane % BL;
    const uint32_t br = sd.row;
    float acc[4][KB];
#pragma unroll
    for (int li = 0; li < 4; ++li)
#pragma unroll
        for (int k = 0; k < KB; ++k) acc[li][k] = 0.0f;
    uint32_t pos = sd.byte_begin, carry = sd.base_col, ebase = sd.elem_begin;
    const uint32_t end = sd.byte_end;
    float *sw = s_w[wave];
    while (pos < end) {
        const Chunk ch = decode_chunk(a.idx, pos, end, carry);
        if (ch.T == 0ull) break;
        if (ch.term) {
            s_bc[wave][ch.rank] = ch.col;
            s_t[wave][ch.rank] = ebase + ch.rank;
        }
        wave_lds_sync();
        const uint32_t n = (uint32_t)__popcll(ch.T);
        // dequantise the window's tiles once: lane q -> (tile q/16, slot q%16)
        for (uint32_t q = lane; q < n * 16u; q += 64u) {
            const uint32_t jt = q >> 4, slot = q & 15u, li = slot & 3u, lj = slot >> 2;
            const uint32_t bc = s_bc[wave][jt];
            const uint32_t byte = a.tiles[(size_t)s_t[wave][jt] * 16u + slot];
            const uint32_t r = br * 4u + li, c = bc * 4u + lj;
            float w = 0.0f;
            if (r < a.rows && c < a.cols) w = fp4_decode(byte & 0xFu) * scale_at(a.sc, r, c);
            if constexpr (SKIP == SKIP_POSZERO) {
                if (byte == 0u) w = __builtin_bit_cast(float, 0xFFFFFFFFu);  // dead-slot marker
            }
            sw[q] = w;
        }
        wave_lds_sync();
        for (uint32_t j = 0; j < n; j += G) {
            const uint32_t e = j + g;
            if (e < n) {
                const uint32_t bc = s_bc[wave][e];
                const float4 *wp = reinterpret_cast<const float4 *>(sw + e * 16u);
                const float4 w0 = wp[0], w1 = wp[1], w2 = wp[2], w3 = wp[3];
                const float wv[4][4] = {{w0.x, w0.y, w0.z, w0.w}, {w1.x, w1.y, w1.z, w1.w},
                                        {w2.x, w2.y, w2.z, w2.w}, {w3.x, w3.y, w3.z, w3.w}};
#pragma unroll
                for (uint32_t lj = 0; lj < 4u; ++lj) {
                    const uint32_t c = bc * 4u + lj;
                    if (c >= a.cols) continue;
                    const float *src = a.in + (int64_t)c * a.in_ld;
#pragma unroll
                    for (int k = 0; k < KB; ++k) {
                        const int64_t b = (int64_t)bl + (int64_t)BL * k;
                        if (b < a.nb) {
                            const float x = src[b];
#pragma unroll
                            for (int li = 0; li < 4; ++li) {
                                const float w = wv[lj][li];
                                if constexpr (SKIP == SKIP_POSZERO) {
                                    if (__builtin_bit_cast(uint32_t, w) == 0xFFFFFFFFu || skip_x<SKIP>(x)) continue;
                                } else if constexpr (SKIP == SKIP_ZERO) {
                                    if (skip_x<SKIP>(x)) continue;
                                }
                                acc[li][k] = __builtin_fmaf(w, x, acc[li][k]);
                            }
                        }
                    }
                }
            }
        }
        wave_lds_sync();
        carry = chunk_advance(ch, pos, ebase);
    }
#pragma unroll
    for (int li = 0; li < 4; ++li) {
        if constexpr (G > 1) {
#pragma unroll
            for (uint32_t off = BL; off < 64u; off <<= 1) acc[li][0] += __shfl_xor(acc[li][0], (int)off, 64);
        }
        const uint32_t r = br * 4u + (uint32_t)li;
        if (g == 0 && r < a.rows) {
#pragma unroll
            for (int k = 0; k < KB; ++k) {
                const int64_t b = (int64_t)bl + (int64_t)BL * k;
                if (b < a.nb) {
                    float *o = a.out + b * a.out_ld + r;
                    if (sd.split & SEG_SPLIT) atomicAdd(o, acc[li][k]);
                    else *o += acc[li][k];
                }
            }
        }
    }
}

struct SArgs {
    const SegDesc *seg;
    int64_t nseg;
    const uint8_t *idx;
    const float *xT;
    const float *gT;
    int64_t B;
    float *gw;
    float *acc_in;  // optional: acc_in[row] += sum_b |xT[row,b]| (first segment of each row)
    uint32_t gT_bytes;  // readable bytes from gT (buffer range for the fast kernel)
};

// acc += sum_b x[b]*g[b] over B floats (B % 4 == 0, 16-byte aligned), with
// four float4 loads in flight.
__device__ __forceinline__ float dot_f4(const float *__restrict__ x, const float *__restrict__ g, int64_t B) {
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
    int64_t b = 0;
    for (; b + 16 <= B; b += 16) {
        const float4 g0 = *reinterpret_cast<const float4 *>(g + b);
        const float4 g1 = *reinterpret_cast<const float4 *>(g + b + 4);
        const float4 g2 = *reinterpret_cast<const float4 *>(g + b + 8);
        const float4 g3 = *reinterpret_cast<const float4 *>(g + b + 12);
        const float4 x0 = *reinterpret_cast<const float4 *>(x + b);
        const float4 x1 = *reinterpret_cast<const float4 *>(x + b + 4);
        const float4 x2 = *reinterpret_cast<const float4 *>(x + b + 8);
        const float4 x3 = *reinterpret_cast<const float4 *>(x + b + 12);
        a0 = __builtin_fmaf(x0.x, g0.x, a0); a1 = __builtin_fmaf(x0.y, g0.y, a1);
        a2 = __builtin_fmaf(x0.z, g0.z, a2); a3 = __builtin_fmaf(x0.w, g0.w, a3);
        a0 = __builtin_fmaf(x1.x, g1.x, a0); a1 = __builtin_fmaf(x1.y, g1.y, a1);
        a2 = __builtin_fmaf(x1.z, g1.z, a2); a3 = __builtin_fmaf(x1.w, g1.w, a3);
        a0 = __builtin_fmaf(x2.x, g2.x, a0); a1 = __builtin_fmaf(x2.y, g2.y, a1);
        a2 = __builtin_fmaf(x2.z, g2.z, a2); a3 = __builtin_fmaf(x2.w, g2.w, a3);
        a0 = __builtin_fmaf(x3.x, g3.x, a0); a1 = __builtin_fmaf(x3.y, g3.y, a1);
        a2 = __builtin_fmaf(x3.z, g3.z, a2); a3 = __builtin_fmaf(x3.w, g3.w, a3);
    }
    for (; b < B; b += 4) {
        const float4 gv = *reinterpret_cast<const float4 *>(g + b);
        const float4 xv = *reinterpret_cast<const float4 *>(x + b);
        a0 = __builtin_fmaf(xv.x, gv.x, a0); a1 = __builtin_fmaf(xv.y, gv.y, a1);
        a2 = __builtin_fmaf(xv.z, gv.z, a2); a3 = __builtin_fmaf(xv.w, gv.w, a3);
    }
    return (a0 + a1) + (a2 + a3);
}

// gw[e] = sum_b xT[row,b] * gT[col_e,b]; each terminator lane owns one entry
// and streams its gT row (float4 along b), xT[row,:] is staged in LDS.
__global__ __launch_bounds__(256) void k_sddmm(SArgs a) {
    extern __shared__ __align__(16) float s_x[];  // [WAVES][B]
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    __shared__ SegStage s_stage[WAVES];
    const int64_t si = (int64_t)blockIdx.x * WAVES + wave;
    if (si >= a.nseg) return;
    const SegDesc sd = a.seg[si];
    const int64_t B = a.B;
    float *sx = s_x + (int64_t)wave * B;
    float part = 0.0f;
    for (int64_t b = lane; b < B; b += 64) {
        const float v = a.xT[(int64_t)sd.row * B + b];
        sx[b] = v;
        part += __builtin_fabsf(v);
    }
    if (a.acc_in && (sd.split & SEG_FIRST)) {
        part = wave_sum(part);
        if (lane == 0) a.acc_in[sd.row] += part;
    }
    wave_lds_sync();
    const StagedSeg sg = stage_segment(s_stage[wave], a.idx, nullptr, sd);
    uint32_t pos = 0, carry = sd.base_col, ebase = sd.elem_begin;
    const uint32_t end = sg.end;
    const bool vec4 = (B & 3) == 0;
    while (pos < end) {
        const Chunk ch = decode_chunk(sg.idx, pos, end, carry);
        if (ch.T == 0ull) break;
        if (ch.term) {
            const float *gr = a.gT + (int64_t)ch.col * B;
            float acc = 0.0f;
            if (vec4) {
                acc = dot_f4(sx, gr, B);
            } else {
                for (int64_t b = 0; b < B; ++b) acc = __builtin_fmaf(sx[b], gr[b], acc);
            }
            a.gw[ebase + ch.rank] = acc;
        }
        carry = chunk_advance(ch, pos, ebase);
    }
}

// Grad-W with float4 along the batch: BL lanes per entry (G = 64/BL entries
// per load instruction), each lane owning float4 chunks q = bl + BL*k of
// both xT[row] (held in registers for the whole segment) and gT[col];
// DPP row reductions finish each entry.  The segment is decoded first into
// an LDS table of gT byte offsets (padding: out of range, loads read 0).
// Needs B % 4 == 0 and 16-byte aligned xT / gT.
template <int BL, int KB, int U>
__global__ __launch_bounds__(256) void k_sddmm_v4(SArgs a) {
    __shared__ SegStage s_stage[WAVES];
    __shared__ uint32_t s_off[WAVES][ENT_CAP];
    constexpr uint32_t G = 64u / BL;
    constexpr uint32_t STEP = G * U;
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const int64_t si = (int64_t)blockIdx.x * WAVES + wave;
    if (si >= a.nseg) return;
    const SegDesc sd = a.seg[si];
    const uint32_t g = lane / BL, bl = lane % BL;
    const uint32_t nq = (uint32_t)(a.B >> 2);
    const uint32_t ld_bytes = (uint32_t)a.B * 4u;
    const float4 *x4p = reinterpret_cast<const float4 *>(a.xT) + (int64_t)sd.row * nq;
    const __amdgpu_buffer_rsrc_t rg = buffer_rsrc(a.gT, a.gT_bytes);
    uint32_t lane_off[KB];
    float4 xr[KB];
    float part = 0.0f;
#pragma unroll
    for (int k = 0; k < KB; ++k) {
        const uint32_t q = bl + BL * (uint32_t)k;
        lane_off[k] = q < nq ? q * 16u : OOB_OFFSET;
        xr[k] = q < nq ? x4p[q] : make_float4(0.f, 0.f, 0.f, 0.f);
        part += (__builtin_fabsf(xr[k].x) + __builtin_fabsf(xr[k].y)) +
                (__builtin_fabsf(xr[k].z) + __builtin_fabsf(xr[k].w));
    }
    if (a.acc_in && (sd.split & SEG_FIRST)) {
        part = group_sum_last<BL>(part);  // every group holds the whole row; use group 0
        if (lane == BL - 1u) a.acc_in[sd.row] += part;
    }
    const StagedSeg sg = stage_segment(s_stage[wave], a.idx, nullptr, sd);
    uint32_t *offs = s_off[wave];
    uint32_t pos = 0, carry = sd.base_col, ebase = sd.elem_begin;
    while (pos < sg.end) {
        const Chunk ch = decode_chunk(sg.idx, pos, sg.end, carry);
        if (ch.T == 0ull) break;
        if (ch.term) offs[ebase - sd.elem_begin + ch.rank] = ch.col * ld_bytes;
        carry = chunk_advance(ch, pos, ebase);
    }
    const uint32_t n = ebase - sd.elem_begin;
    const uint32_t npad = (n + STEP - 1u) / STEP * STEP;
    for (uint32_t k = n + lane; k < npad; k += 64u) offs[k] = OOB_OFFSET;
    wave_lds_sync();
    for (uint32_t j = 0; j < n; j += STEP) {
        float4 gv[U][KB];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t off = offs[j + (uint32_t)u * G + g];
#pragma unroll
            for (int k = 0; k < KB; ++k) gv[u][k] = buffer_load_f4(rg, off + lane_off[k]);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float d0 = 0.f, d1 = 0.f;
#pragma unroll
            for (int k = 0; k < KB; ++k) {
                d0 = __builtin_fmaf(xr[k].x, gv[u][k].x, d0);
                d1 = __builtin_fmaf(xr[k].y, gv[u][k].y, d1);
                d0 = __builtin_fmaf(xr[k].z, gv[u][k].z, d0);
                d1 = __builtin_fmaf(xr[k].w, gv[u][k].w, d1);
            }
            const float tot = group_sum_last<BL>(d0 + d1);
            const uint32_t e = j + (uint32_t)u * G + g;
            if (bl == BL - 1u && e < n) a.gw[sd.elem_begin + e] = tot;
        }
    }
}

struct FArgs {
    const SegDesc *seg;
    int64_t nseg;
    const uint8_t *idx;
    const uint8_t *val;
    ScaleView sc;
    const float *gT;    // [cols, B] feature-major upstream gradient
    uint32_t gT_bytes;
    const float *xT;    // [rows, B] feature-major forward input
    int64_t B;
    float *dx;          // [B, dx_ld] batch-major
    int64_t dx_ld;
    float *gw;          // one value per stored synapse, elem order
    float *acc_in;      // optional: acc_in[row] += sum_b |xT[row,b]|
    int xcd;            // XCD-contiguous block order (xcd_block)
    // split rows of dx combined in order by their last item (GatherPlan)
    const uint32_t *elem_start;
    uint32_t *split_cnt;
    float *part;
};

// Fused grad-input + nnz-sampled grad-W over the canonical store: one decode
// of the segment, one load of gT[col] per entry, used twice --
//   dx[b,row] += w_e * gT[col_e,b]        (the grad-input gather)
//   gw[e]      = sum_b xT[row,b]*gT[col_e,b] (the sampled grad-W)
// Lane layout as k_gather_v4 (BL lanes per entry, float4 chunks of the
// batch), xT[row] in registers as k_sddmm_v4.  Needs B % 4 == 0, 16-byte
// aligned xT / gT and B <= 64*KB*4/ (64/BL) -- the launcher checks.
template <int BL, int KB, int U>
__global__ __attribute__((amdgpu_flat_work_group_size(1, 256), amdgpu_waves_per_eu(KB <= 2 && KB * U <= 4 ? 8 : 1)))
void k_bwd_v4(FArgs a) {
    __shared__ SegStage s_stage[WAVES];
    __shared__ uint2 s_ent[WAVES][ENT_CAP];
    __shared__ float s_fp4[WAVES][16];
    constexpr uint32_t G = 64u / BL;
    constexpr uint32_t STEP = G * U;
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const uint32_t bid = a.xcd ? xcd_block(blockIdx.x, gridDim.x) : blockIdx.x;
    const int64_t si = (int64_t)bid * WAVES + wave;
    const bool active = si < a.nseg;  // inactive waves still join the block epilogue
    const uint32_t g = lane / BL, bl = lane % BL;
    const uint32_t nq = (uint32_t)(a.B >> 2);
    float4 acc[KB];
#pragma unroll
    for (int k = 0; k < KB; ++k) acc[k] = make_float4(0.f, 0.f, 0.f, 0.f);
    SegDesc sd{};
    if (active) {
    sd = a.seg[si];
    fp4_table_init(s_fp4[wave]);
    const StagedSeg sg = stage_segment(s_stage[wave], a.idx, a.val, sd);
    const __amdgpu_buffer_rsrc_t rg = buffer_rsrc(a.gT, a.gT_bytes);
    const float4 *x4p = reinterpret_cast<const float4 *>(a.xT) + (int64_t)sd.row * nq;
    uint32_t lane_off[KB];
    float4 xr[KB];
    float part = 0.0f;
#pragma unroll
    for (int k = 0; k < KB; ++k) {
        const uint32_t q = bl + BL * (uint32_t)k;
        lane_off[k] = q < nq ? q * 16u : OOB_OFFSET;
        xr[k] = q < nq ? x4p[q] : make_float4(0.f, 0.f, 0.f, 0.f);
        part += (__builtin_fabsf(xr[k].x) + __builtin_fabsf(xr[k].y)) +
                (__builtin_fabsf(xr[k].z) + __builtin_fabsf(xr[k].w));
    }
    if (a.acc_in && (sd.split & SEG_FIRST)) {
        part = group_sum_last<BL>(part);  // every group holds the whole row; use group 0
        if (lane == BL - 1u) a.acc_in[sd.row] += part;
    }
    uint2 *ent = s_ent[wave];
    const uint32_t n = decode_segment_entries(sg, sd, a.sc, s_fp4[wave], (uint32_t)a.B * 4u, STEP, ent);
    for (uint32_t j = 0; j < n; j += STEP) {
        uint2 e[U];
        float4 gv[U][KB];
#pragma unroll
        for (int u = 0; u < U; ++u) e[u] = ent[j + (uint32_t)u * G + g];
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int k = 0; k < KB; ++k) gv[u][k] = buffer_load_f4(rg, e[u].x + lane_off[k]);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const float w = __builtin_bit_cast(float, e[u].y);
            float d0 = 0.f, d1 = 0.f;
#pragma unroll
            for (int k = 0; k < KB; ++k) {
                acc[k].x = __builtin_fmaf(w, gv[u][k].x, acc[k].x);
                acc[k].y = __builtin_fmaf(w, gv[u][k].y, acc[k].y);
                acc[k].z = __builtin_fmaf(w, gv[u][k].z, acc[k].z);
                acc[k].w = __builtin_fmaf(w, gv[u][k].w, acc[k].w);
                d0 = __builtin_fmaf(xr[k].x, gv[u][k].x, d0);
                d1 = __builtin_fmaf(xr[k].y, gv[u][k].y, d1);
                d0 = __builtin_fmaf(xr[k].z, gv[u][k].z, d0);
                d1 = __builtin_fmaf(xr[k].w, gv[u][k].w, d1);
            }
            const float tot = group_sum_last<BL>(d0 + d1);
            const uint32_t ei = j + (uint32_t)u * G + g;
            if (bl == BL - 1u && ei < n) a.gw[sd.elem_begin + ei] = tot;
        }
    }
#pragma unroll
    for (uint32_t off = BL; off < 64u; off <<= 1)
#pragma unroll
        for (int k = 0; k < KB; ++k) {
            acc[k].x += __shfl_xor(acc[k].x, (int)off, 64);
            acc[k].y += __shfl_xor(acc[k].y, (int)off, 64);
            acc[k].z += __shfl_xor(acc[k].z, (int)off, 64);
            acc[k].w += __shfl_xor(acc[k].w, (int)off, 64);
        }
    wave_lds_sync();  // the entry table is reused as this wave's output slice
    }
    store_rows_block<BL, KB>(acc, active, sd.row, (sd.split & SEG_SPLIT) != 0, nq,
                             reinterpret_cast<float *>(&s_ent[0][0]), ENT_CAP * 2u, a.dx, a.dx_ld, false,
                             SplitCombine{a.seg, a.nseg, a.elem_start, a.split_cnt, a.part}, si,
                             sd.elem_end - sd.elem_begin);
}

// Block epilogue for block4 waves: out[b, 4*brow+li] for the block's (up to
// WAVES) segments over one batch chunk [b0, b0 + nbc).  Each wave leaves its
// results in its LDS slice, row li at li * row_stride; the block then writes them
// with consecutive lanes on consecutive rows (the 4*WAVES rows of one batch
// index form one run when the block rows are consecutive).  The results
// add to out (the scattered pass wrote it first); split rows add
// atomically.  Every thread of the block calls this.
__device__ __forceinline__ void store_rows4_block(bool active, uint32_t brow, bool split, uint32_t b0,
                                                  uint32_t nbc, uint32_t row_stride, const float *slice_base,
                                                  uint32_t slice_stride, int64_t rows, float *out, int64_t out_ld) {
    __shared__ uint32_t s_brow[WAVES];
    __shared__ uint32_t s_flag[WAVES];
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    if (lane == 0) {
        s_brow[wave] = brow;
        s_flag[wave] = (active ? 1u : 0u) | (split ? 2u : 0u);
    }
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < nbc * 4u * WAVES; i += blockDim.x) {
        const uint32_t li = i & 3u, w = (i >> 2) % WAVES, b = i / (4u * WAVES);
        const uint32_t f = s_flag[w];
        const int64_t r = (int64_t)s_brow[w] * 4 + li;
        if (!(f & 1u) || r >= rows) continue;
        const float v = slice_base[w * slice_stride + li * row_stride + b];
        float *o = out + (int64_t)(b0 + b) * out_ld + r;
        if (f & 2u) atomicAdd(o, v);
        else *o += v;
    }
}

// Block4 gather with float4 batch lanes (dense paths, no skip rules): one
// wave per (segment, batch chunk of 4*BL*KB columns -- blockIdx.y).  The
// segment's block-column deltas are decoded 64 at a time; the lane that
// decodes a tile dequantises its 16 slots into LDS (one 16-byte tile load);
// then G = 64/BL tiles per load instruction, U tiles per group in flight,
// each lane loading the 4 input rows 4bc+lj of its tile (float4 chunks of
// the batch) and accumulating the tile's 4 output rows.  Needs nb % 4 == 0,
// in_ld % 4 == 0, a 16-byte aligned `in` and a < 2 GiB input.
template <int BL, int KB, int U>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(U <= 2 ? 4 : 1))) void k_gather_b4_v4(BArgs a, uint32_t in_bytes) {
    __shared__ uint32_t s_off[WAVES][64];
    __shared__ __align__(16) float s_w[WAVES][64 * 16];
    __shared__ float s_fp4[WAVES][16];
    constexpr uint32_t G = 64u / BL;
    constexpr uint32_t STEP = G * U;
    constexpr uint32_t NBC = 4u * BL * KB;  // batch columns per wave
    static_assert(4u * NBC <= 64u * 16u, "output slice must fit the weight table");
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    uint32_t bx = blockIdx.x, by = blockIdx.y;
    if (a.xq_gx) {
        const uint32_t lb = xcd_block(blockIdx.x, gridDim.x);
        by = lb / a.xq_gx;
        bx = lb % a.xq_gx;
    }
    const int64_t si = (int64_t)bx * WAVES + wave;
    const bool active = si < a.nseg;
    const uint32_t g = lane / BL, bl = lane % BL;
    const uint32_t nq = (uint32_t)(a.nb >> 2);
    const uint32_t q0 = by * (BL * KB);
    float4 acc[4][KB];
#pragma unroll
    for (int li = 0; li < 4; ++li)
#pragma unroll
        for (int k = 0; k < KB; ++k) acc[li][k] = make_float4(0.f, 0.f, 0.f, 0.f);
    SegDesc sd{};
    if (active) {
    sd = a.seg[si];
    const uint32_t br = sd.row;
    const __amdgpu_buffer_rsrc_t rin = buffer_rsrc(a.in, in_bytes);
    const uint32_t ld_bytes = (uint32_t)a.in_ld * 4u;
    uint32_t lane_off[KB];
#pragma unroll
    for (int k = 0; k < KB; ++k) {
        const uint32_t q = q0 + bl + BL * (uint32_t)k;
        lane_off[k] = q < nq ? q * 16u : OOB_OFFSET;
    }
    float *sw = s_w[wave];
    fp4_table_init(s_fp4[wave]);
    wave_lds_sync();
    const float *tab = s_fp4[wave];
    // rank-1 scales of the block row's 4 rows (uniform over the segment)
    float rs[4];
#pragma unroll
    for (int li = 0; li < 4; ++li) {
        const uint32_t r = br * 4u + (uint32_t)li;
        rs[li] = (a.sc.row && r < a.rows) ? a.sc.row[r] : 1.0f;
    }
    uint32_t pos = sd.byte_begin, carry = sd.base_col, ebase = sd.elem_begin;
    const uint32_t end = sd.byte_end;
    while (pos < end) {
        const Chunk ch = decode_chunk(a.idx, pos, end, carry);
        if (ch.T == 0ull) break;
        const uint32_t n = (uint32_t)__popcll(ch.T);
        const uint32_t npad = (n + STEP - 1u) / STEP * STEP;
        if (ch.term) {
            // the lane that decoded tile `rank` dequantises its 16 slots:
            // one 16-byte load of the tile, scales S(r,c) as scale_at; the
            // scale rank is one uniform branch here (a per-slot choice would
            // carry scale_at's loop into every slot), codes by the LDS table
            const uint32_t bc = ch.col;
            s_off[wave][ch.rank] = bc * 4u * ld_bytes;
            const uint4 tb = *reinterpret_cast<const uint4 *>(a.tiles + (size_t)(ebase + ch.rank) * 16u);
            const uint32_t words[4] = {tb.x, tb.y, tb.z, tb.w};  // word lj holds slots lj*4 .. lj*4+3
            bool rok[4];
#pragma unroll
            for (int li = 0; li < 4; ++li) rok[li] = br * 4u + (uint32_t)li < a.rows;
            if (a.sc.rank == 1) {
                float cs[4];
#pragma unroll
                for (int lj = 0; lj < 4; ++lj) {
                    const uint32_t c = bc * 4u + (uint32_t)lj;
                    cs[lj] = (a.sc.ent && c < a.cols) ? a.sc.ent[c] : 1.0f;
                }
#pragma unroll
                for (int lj = 0; lj < 4; ++lj) {
                    const bool cok = bc * 4u + (uint32_t)lj < a.cols;
                    float wv[4];
#pragma unroll
                    for (int li = 0; li < 4; ++li) {
                        const float S = a.sc.ent ? rs[li] * cs[lj] : rs[li];
                        const float d = tab[(words[lj] >> (8 * li)) & 0xFu];
                        wv[li] = (rok[li] && cok) ? d * S : 0.0f;
                    }
                    reinterpret_cast<float4 *>(sw + ch.rank * 16u)[lj] = make_float4(wv[0], wv[1], wv[2], wv[3]);
                }
            } else {
#pragma unroll
                for (int lj = 0; lj < 4; ++lj) {
                    const uint32_t c = bc * 4u + (uint32_t)lj;
                    const bool cok = c < a.cols;
                    float wv[4];
#pragma unroll
                    for (int li = 0; li < 4; ++li) {
                        const uint32_t r = br * 4u + (uint32_t)li;
                        const float S = (rok[li] && cok) ? scale_at(a.sc, r, c) : 1.0f;
                        const float d = tab[(words[lj] >> (8 * li)) & 0xFu];
                        wv[li] = (rok[li] && cok) ? d * S : 0.0f;
                    }
                    reinterpret_cast<float4 *>(sw + ch.rank * 16u)[lj] = make_float4(wv[0], wv[1], wv[2], wv[3]);
                }
            }
        }
        // padding slots n .. npad-1 (a terminator lane can sit at or past n when
        // a varint spans several bytes, so every lane checks)
        if (lane >= n && lane < npad) {
            // padding tiles: out-of-range rows (read 0), zero weights
            s_off[wave][lane] = OOB_OFFSET;
#pragma unroll
            for (int lj = 0; lj < 4; ++lj)
                reinterpret_cast<float4 *>(sw + lane * 16u)[lj] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
        wave_lds_sync();
        for (uint32_t j = 0; j < npad; j += STEP) {
            float4 x[U][4][KB];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const uint32_t off = s_off[wave][j + (uint32_t)u * G + g];
#pragma unroll
                for (int lj = 0; lj < 4; ++lj)
#pragma unroll
                    for (int k = 0; k < KB; ++k)
                        x[u][lj][k] = buffer_load_f4(rin, off + (uint32_t)lj * ld_bytes + lane_off[k]);
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const float4 *wp = reinterpret_cast<const float4 *>(sw + (j + (uint32_t)u * G + g) * 16u);
                const float4 wv[4] = {wp[0], wp[1], wp[2], wp[3]};  // wv[lj] = slots (lj, li = 0..3)
#pragma unroll
                for (int lj = 0; lj < 4; ++lj) {
                    const float wl[4] = {wv[lj].x, wv[lj].y, wv[lj].z, wv[lj].w};
#pragma unroll
                    for (int li = 0; li < 4; ++li)
#pragma unroll
                        for (int k = 0; k < KB; ++k) {
                            acc[li][k].x = __builtin_fmaf(wl[li], x[u][lj][k].x, acc[li][k].x);
                            acc[li][k].y = __builtin_fmaf(wl[li], x[u][lj][k].y, acc[li][k].y);
                            acc[li][k].z = __builtin_fmaf(wl[li], x[u][lj][k].z, acc[li][k].z);
                            acc[li][k].w = __builtin_fmaf(wl[li], x[u][lj][k].w, acc[li][k].w);
                        }
                }
            }
        }
        wave_lds_sync();
        carry = chunk_advance(ch, pos, ebase);
    }
    // combine the G tile groups (lanes bl, bl+BL, ...)
#pragma unroll
    for (uint32_t off = BL; off < 64u; off <<= 1)
#pragma unroll
        for (int li = 0; li < 4; ++li)
#pragma unroll
            for (int k = 0; k < KB; ++k) {
                acc[li][k].x += __shfl_xor(acc[li][k].x, (int)off, 64);
                acc[li][k].y += __shfl_xor(acc[li][k].y, (int)off, 64);
                acc[li][k].z += __shfl_xor(acc[li][k].z, (int)off, 64);
                acc[li][k].w += __shfl_xor(acc[li][k].w, (int)off, 64);
            }
    // this wave's slice of the weight table now holds its 4 x NBC results
    if (g == 0) {
#pragma unroll
        for (int li = 0; li < 4; ++li)
#pragma unroll
            for (int k = 0; k < KB; ++k)
                reinterpret_cast<float4 *>(sw + (uint32_t)li * NBC)[bl + BL * (uint32_t)k] = acc[li][k];
    }
    }
    const uint32_t b0 = q0 * 4u;
    const uint32_t nbc = (uint32_t)a.nb > b0 ? ((uint32_t)a.nb - b0 < NBC ? (uint32_t)a.nb - b0 : NBC) : 0u;
    store_rows4_block(active, sd.row, (sd.split & SEG_SPLIT) != 0, b0, nbc, NBC, &s_w[0][0], 64u * 16u, a.rows,
                      a.out, a.out_ld);
}

struct SBArgs {
    const SegDesc *seg;
    int64_t nseg;
    const uint8_t *idx;
    int64_t rows, cols;
    const float *xT;
    const float *gT;
    int64_t B;
    float *gw;
};

// Block4 gather, one tile per wave step: lane (lj = lane/16, bl = lane%16)
// loads float4 chunk bl of input row 4bc+lj (64 batch columns per wave --
// blockIdx.y) and accumulates the tile's 4 output rows with the 4 weights
// (lj, li = 0..3); the 4 lj groups are summed once per segment.  U tiles in
// flight per lane.  Same preconditions as k_gather_b4_v4 with
// nb >= 64 columns per chunk layout (16 float4 per wave).
template <int U>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(6))) void k_gather_b4_w(BArgs a, uint32_t in_bytes) {
    __shared__ uint32_t s_off[WAVES][64];
    __shared__ __align__(16) float s_w[WAVES][64 * 16];
    constexpr uint32_t NBC = 64u;  // batch columns per wave
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const int64_t si = (int64_t)blockIdx.x * WAVES + wave;
    const bool active = si < a.nseg;
    const uint32_t lj = lane >> 4, bl = lane & 15u;
    const uint32_t nq = (uint32_t)(a.nb >> 2);
    const uint32_t q0 = blockIdx.y * 16u;
    float4 acc[4];
#pragma unroll
    for (int li = 0; li < 4; ++li) acc[li] = make_float4(0.f, 0.f, 0.f, 0.f);
    SegDesc sd{};
    float *sw = s_w[wave];
    if (active) {
    sd = a.seg[si];
    const uint32_t br = sd.row;
    const __amdgpu_buffer_rsrc_t rin = buffer_rsrc(a.in, in_bytes);
    const uint32_t ld_bytes = (uint32_t)a.in_ld * 4u;
    const uint32_t q = q0 + bl;
    const uint32_t lane_off = (q < nq ? q * 16u : OOB_OFFSET);
    const uint32_t row_off = lj * ld_bytes;
    float rs[4];
#pragma unroll
    for (int li = 0; li < 4; ++li) {
        const uint32_t r = br * 4u + (uint32_t)li;
        rs[li] = (a.sc.row && r < a.rows) ? a.sc.row[r] : 1.0f;
    }
    uint32_t pos = sd.byte_begin, carry = sd.base_col, ebase = sd.elem_begin;
    const uint32_t end = sd.byte_end;
    while (pos < end) {
        const Chunk ch = decode_chunk(a.idx, pos, end, carry);
        if (ch.T == 0ull) break;
        const uint32_t n = (uint32_t)__popcll(ch.T);
        const uint32_t npad = (n + U - 1u) / U * U;
        if (ch.term) {
            const uint32_t bc = ch.col;
            s_off[wave][ch.rank] = bc * 4u * ld_bytes;
            const uint4 tb = *reinterpret_cast<const uint4 *>(a.tiles + (size_t)(ebase + ch.rank) * 16u);
            const uint32_t words[4] = {tb.x, tb.y, tb.z, tb.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t c = bc * 4u + (uint32_t)j;
                const bool cok = c < a.cols;
                const float cs = (a.sc.rank == 1 && a.sc.ent && cok) ? a.sc.ent[c] : 1.0f;
                float wv[4];
#pragma unroll
                for (int li = 0; li < 4; ++li) {
                    const uint32_t r = br * 4u + (uint32_t)li;
                    const uint32_t code = (words[j] >> (8 * li)) & 0xFu;
                    float S;
                    if (a.sc.rank == 1) S = a.sc.ent ? rs[li] * cs : rs[li];
                    else S = (r < a.rows && cok) ? scale_at(a.sc, r, c) : 1.0f;
                    wv[li] = (r < a.rows && cok) ? fp4_decode(code) * S : 0.0f;
                }
                reinterpret_cast<float4 *>(sw + ch.rank * 16u)[j] = make_float4(wv[0], wv[1], wv[2], wv[3]);
            }
        }
        // padding slots n .. npad-1 (a terminator lane can sit at or past n when
        // a varint spans several bytes, so every lane checks)
        if (lane >= n && lane < npad) {
            s_off[wave][lane] = OOB_OFFSET;
#pragma unroll
            for (int j = 0; j < 4; ++j)
                reinterpret_cast<float4 *>(sw + lane * 16u)[j] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
        wave_lds_sync();
        for (uint32_t e0 = 0; e0 < npad; e0 += U) {
            float4 x[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const uint32_t off = s_off[wave][e0 + (uint32_t)u];
                x[u] = buffer_load_f4(rin, (off == OOB_OFFSET ? OOB_OFFSET : off + row_off) + lane_off);
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const float4 w = reinterpret_cast<const float4 *>(sw + (e0 + (uint32_t)u) * 16u)[lj];
                const float wl[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
                for (int li = 0; li < 4; ++li) {
                    acc[li].x = __builtin_fmaf(wl[li], x[u].x, acc[li].x);
                    acc[li].y = __builtin_fmaf(wl[li], x[u].y, acc[li].y);
                    acc[li].z = __builtin_fmaf(wl[li], x[u].z, acc[li].z);
                    acc[li].w = __builtin_fmaf(wl[li], x[u].w, acc[li].w);
                }
            }
        }
        wave_lds_sync();
        carry = chunk_advance(ch, pos, ebase);
    }
    // sum the 4 input-row groups (lanes bl, bl+16, bl+32, bl+48)
#pragma unroll
    for (uint32_t off = 16u; off < 64u; off <<= 1)
#pragma unroll
        for (int li = 0; li < 4; ++li) {
            acc[li].x += __shfl_xor(acc[li].x, (int)off, 64);
            acc[li].y += __shfl_xor(acc[li].y, (int)off, 64);
            acc[li].z += __shfl_xor(acc[li].z, (int)off, 64);
            acc[li].w += __shfl_xor(acc[li].w, (int)off, 64);
        }
    if (lj == 0) {
#pragma unroll
        for (int li = 0; li < 4; ++li) reinterpret_cast<float4 *>(sw + (uint32_t)li * NBC)[bl] = acc[li];
    }
    }
    const uint32_t b0 = q0 * 4u;
    const uint32_t nbc = (uint32_t)a.nb > b0 ? ((uint32_t)a.nb - b0 < NBC ? (uint32_t)a.nb - b0 : NBC) : 0u;
    store_rows4_block(active, sd.row, (sd.split & SEG_SPLIT) != 0, b0, nbc, NBC, &s_w[0][0], 64u * 16u, a.rows,
                      a.out, a.out_ld);
}

typedef float v4f __attribute__((ext_vector_type(4)));

// Block4 gather on the matrix cores: one wave per (segment, 64 batch
// columns b0 = 64*blockIdx.y); lane l owns batch column b0+l.  With
// v_mfma_f32_4x4x1 (16 blocks of D[4x4] += A[4x1]*B[1x4]; block b = lane/4,
// A[b][i] from lane 4b+i, B[b][j] from lane 4b+j, D[b][i][j] in vgpr i of
// lane 4b+j) the blocks are 16 groups of 4 batch columns: A = column lj of
// the tile's weights (lane 4b+i: W[i][lj]), B = input row 4bc+lj (lane l:
// x[4bc+lj][b0+l]), so vgpr li of lane l accumulates out[4br+li][b0+l].
// 4 MFMAs per tile (one accumulator per lj), U tiles in flight.  Same
// preconditions as k_gather_b4_v4.
template <int U>
__global__ __launch_bounds__(256) void k_gather_b4_mfma(BArgs a, uint32_t in_bytes) {
    __shared__ uint32_t s_off[WAVES][64];
    __shared__ __align__(16) float s_w[WAVES][64 * 16];  // per tile [li][lj]
    constexpr uint32_t NBC = 64u;
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const int64_t si = (int64_t)blockIdx.x * WAVES + wave;
    const bool active = si < a.nseg;
    const uint32_t b0 = blockIdx.y * NBC;
    v4f acc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] = v4f{0.f, 0.f, 0.f, 0.f};
    SegDesc sd{};
    float *sw = s_w[wave];
    if (active) {
    sd = a.seg[si];
    const uint32_t br = sd.row;
    const __amdgpu_buffer_rsrc_t rin = buffer_rsrc(a.in, in_bytes);
    const uint32_t ld_bytes = (uint32_t)a.in_ld * 4u;
    const uint32_t lane_off = (int64_t)(b0 + lane) < a.nb ? (b0 + lane) * 4u : OOB_OFFSET;
    float rs[4];
#pragma unroll
    for (int li = 0; li < 4; ++li) {
        const uint32_t r = br * 4u + (uint32_t)li;
        rs[li] = (a.sc.row && r < a.rows) ? a.sc.row[r] : 1.0f;
    }
    uint32_t pos = sd.byte_begin, carry = sd.base_col, ebase = sd.elem_begin;
    const uint32_t end = sd.byte_end;
    while (pos < end) {
        const Chunk ch = decode_chunk(a.idx, pos, end, carry);
        if (ch.T == 0ull) break;
        const uint32_t n = (uint32_t)__popcll(ch.T);
        const uint32_t npad = (n + U - 1u) / U * U;
        if (ch.term) {
            const uint32_t bc = ch.col;
            s_off[wave][ch.rank] = bc * 4u * ld_bytes;
            const uint4 tb = *reinterpret_cast<const uint4 *>(a.tiles + (size_t)(ebase + ch.rank) * 16u);
            const uint32_t words[4] = {tb.x, tb.y, tb.z, tb.w};  // word lj holds slots lj*4 .. lj*4+3
            float wm[4][4];                                       // [li][lj]
#pragma unroll
            for (int lj = 0; lj < 4; ++lj) {
                const uint32_t c = bc * 4u + (uint32_t)lj;
                const bool cok = c < a.cols;
                const float cs = (a.sc.rank == 1 && a.sc.ent && cok) ? a.sc.ent[c] : 1.0f;
#pragma unroll
                for (int li = 0; li < 4; ++li) {
                    const uint32_t r = br * 4u + (uint32_t)li;
                    const uint32_t code = (words[lj] >> (8 * li)) & 0xFu;
                    float S;
                    if (a.sc.rank == 1) S = a.sc.ent ? rs[li] * cs : rs[li];
                    else S = (r < a.rows && cok) ? scale_at(a.sc, r, c) : 1.0f;
                    wm[li][lj] = (r < a.rows && cok) ? fp4_decode(code) * S : 0.0f;
                }
            }
#pragma unroll
            for (int li = 0; li < 4; ++li)
                reinterpret_cast<float4 *>(sw + ch.rank * 16u)[li] = make_float4(wm[li][0], wm[li][1], wm[li][2], wm[li][3]);
        }
        // padding slots n .. npad-1 (a terminator lane can sit at or past n when
        // a varint spans several bytes, so every lane checks)
        if (lane >= n && lane < npad) {
            s_off[wave][lane] = OOB_OFFSET;
#pragma unroll
            for (int li = 0; li < 4; ++li)
                reinterpret_cast<float4 *>(sw + lane * 16u)[li] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
        wave_lds_sync();
        for (uint32_t e0 = 0; e0 < npad; e0 += U) {
            float xv[U][4];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const uint32_t off = s_off[wave][e0 + (uint32_t)u];
#pragma unroll
                for (int lj = 0; lj < 4; ++lj)
                    xv[u][lj] = buffer_load_f1(rin, (off == OOB_OFFSET ? OOB_OFFSET : off + (uint32_t)lj * ld_bytes) + lane_off);
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                // A operands: W[lane%4][lj] for lj = 0..3
                const float4 w = reinterpret_cast<const float4 *>(sw + (e0 + (uint32_t)u) * 16u)[lane & 3u];
                acc[0] = __builtin_amdgcn_mfma_f32_4x4x1f32(w.x, xv[u][0], acc[0], 0, 0, 0);
                acc[1] = __builtin_amdgcn_mfma_f32_4x4x1f32(w.y, xv[u][1], acc[1], 0, 0, 0);
                acc[2] = __builtin_amdgcn_mfma_f32_4x4x1f32(w.z, xv[u][2], acc[2], 0, 0, 0);
                acc[3] = __builtin_amdgcn_mfma_f32_4x4x1f32(w.w, xv[u][3], acc[3], 0, 0, 0);
            }
        }
        wave_lds_sync();
        carry = chunk_advance(ch, pos, ebase);
    }
    // this wave's slice of the weight table now holds out[li][b0 + lane]
#pragma unroll
    for (int li = 0; li < 4; ++li)
        sw[(uint32_t)li * NBC + lane] = (acc[0][li] + acc[1][li]) + (acc[2][li] + acc[3][li]);
    }
    const uint32_t nbc = (uint32_t)a.nb > b0 ? ((uint32_t)a.nb - b0 < NBC ? (uint32_t)a.nb - b0 : NBC) : 0u;
    store_rows4_block(active, sd.row, (sd.split & SEG_SPLIT) != 0, b0, nbc, NBC, &s_w[0][0], 64u * 16u, a.rows,
                      a.out, a.out_ld);
}

// Block4 grad-W on the matrix cores: gw[16t + lj*4+li] =
// sum_b xT[4br+li, b] * gT[4bc+lj, b].  One wave per segment over the whole
// batch (B <= 64*KQ).  v_mfma_f32_4x4x1 blocks split the batch: lane
// l = 4*blk + i supplies A = xT[4br+i][n] and B = gT[4bc+i][n] for
// n = 4*(blk + 16s) + c (s < KQ float4 loads, c < 4), so block blk
// accumulates its batch share of the tile's 4x4 product; the 16 blocks are
// summed over lanes with stride 4 (DPP row_shr 4, 8 within 16-lane rows,
// then across rows).  U tiles in flight.  Needs B % 4 == 0 and 16-byte
// aligned xT / gT / gw.
template <int KQ, int U>
__global__ __launch_bounds__(256) void k_sddmm_b4_mfma(SBArgs a, uint32_t gT_bytes) {
    __shared__ uint32_t s_off[WAVES][64];
    __shared__ uint32_t s_t[WAVES][64];
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const int64_t si = (int64_t)blockIdx.x * WAVES + wave;
    if (si >= a.nseg) return;
    const SegDesc sd = a.seg[si];
    const uint32_t li = lane & 3u, blk = lane >> 2;
    const uint32_t nq = (uint32_t)(a.B >> 2);
    const uint32_t ld_bytes = (uint32_t)a.B * 4u;
    const __amdgpu_buffer_rsrc_t rg = buffer_rsrc(a.gT, gT_bytes);
    uint32_t lane_off[KQ];
    float4 xr[KQ];
    const int64_t r = (int64_t)sd.row * 4 + li;
#pragma unroll
    for (int s = 0; s < KQ; ++s) {
        const uint32_t q = blk + 16u * (uint32_t)s;
        lane_off[s] = q < nq ? q * 16u : OOB_OFFSET;
        xr[s] = (q < nq && r < a.rows) ? reinterpret_cast<const float4 *>(a.xT + r * a.B)[q]
                                       : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    const uint32_t row_off = li * ld_bytes;  // this lane supplies gT row 4bc + li
    uint32_t pos = sd.byte_begin, carry = sd.base_col, ebase = sd.elem_begin;
    const uint32_t end = sd.byte_end;
    while (pos < end) {
        const Chunk ch = decode_chunk(a.idx, pos, end, carry);
        if (ch.T == 0ull) break;
        if (ch.term) {
            s_off[wave][ch.rank] = ch.col * 4u * ld_bytes;
            s_t[wave][ch.rank] = ebase + ch.rank;
        }
        wave_lds_sync();
        const uint32_t n = (uint32_t)__popcll(ch.T);
        for (uint32_t e0 = 0; e0 < n; e0 += U) {
            float4 gv[U][KQ];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const uint32_t e = e0 + (uint32_t)u;
                const uint32_t off = e < n ? s_off[wave][e] + row_off : OOB_OFFSET;
#pragma unroll
                for (int s = 0; s < KQ; ++s)
                    gv[u][s] = buffer_load_f4(rg, off == OOB_OFFSET ? OOB_OFFSET : off + lane_off[s]);
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                v4f c0 = {0.f, 0.f, 0.f, 0.f}, c1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int s = 0; s < KQ; ++s) {
                    c0 = __builtin_amdgcn_mfma_f32_4x4x1f32(xr[s].x, gv[u][s].x, c0, 0, 0, 0);
                    c1 = __builtin_amdgcn_mfma_f32_4x4x1f32(xr[s].y, gv[u][s].y, c1, 0, 0, 0);
                    c0 = __builtin_amdgcn_mfma_f32_4x4x1f32(xr[s].z, gv[u][s].z, c0, 0, 0, 0);
                    c1 = __builtin_amdgcn_mfma_f32_4x4x1f32(xr[s].w, gv[u][s].w, c1, 0, 0, 0);
                }
                float d[4];
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    float x = c0[v] + c1[v];
                    x += dpp_f32<DPP_ROW_SHR4>(x);  // lane 12+j of each row: its 4 blocks
                    x += dpp_f32<DPP_ROW_SHR8>(x);
                    x += __shfl_xor(x, 16, 64);     // across the 4 rows
                    x += __shfl_xor(x, 32, 64);
                    d[v] = x;
                }
                const uint32_t e = e0 + (uint32_t)u;
                // lane 12 + j holds D[i = v][j]: slots j*4 + v of tile e
                if (lane >= 12u && lane < 16u && e < n)
                    reinterpret_cast<float4 *>(a.gw + (size_t)s_t[wave][e] * 16u)[lane - 12u] =
                        make_float4(d[0], d[1], d[2], d[3]);
            }
        }
        wave_lds_sync();
        carry = chunk_advance(ch, pos, ebase);
    }
}

// Block4 grad-W with float4 batch lanes: gw[16t + lj*4+li] =
// sum_b xT[4br+li, b] * gT[4bc+lj, b].  One wave per segment over the whole
// batch (B = 4*BL*KB at most): xT's 4 rows of the block row stay in
// registers; G = 64/BL tiles per load instruction, each lane loading the 4
// gT rows of its tile and forming 16 partial dots, reduced over the BL
// batch lanes; the group's last lane stores the tile's 64 bytes.  Needs
// B % 4 == 0, 16-byte aligned xT / gT / gw and a < 2 GiB gT.
template <int BL, int KB>
__global__ __launch_bounds__(256) void k_sddmm_b4_v4(SBArgs a, uint32_t gT_bytes) {
    __shared__ uint32_t s_off[WAVES][64];
    __shared__ uint32_t s_t[WAVES][64];
    constexpr uint32_t G = 64u / BL;
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const int64_t si = (int64_t)blockIdx.x * WAVES + wave;
    if (si >= a.nseg) return;
    const SegDesc sd = a.seg[si];
    const uint32_t g = lane / BL, bl = lane % BL;
    const uint32_t nq = (uint32_t)(a.B >> 2);
    const uint32_t ld_bytes = (uint32_t)a.B * 4u;
    const __amdgpu_buffer_rsrc_t rg = buffer_rsrc(a.gT, gT_bytes);
    uint32_t lane_off[KB];
    float4 xr[4][KB];
#pragma unroll
    for (int k = 0; k < KB; ++k) {
        const uint32_t q = bl + BL * (uint32_t)k;
        lane_off[k] = q < nq ? q * 16u : OOB_OFFSET;
#pragma unroll
        for (int li = 0; li < 4; ++li) {
            const int64_t r = (int64_t)sd.row * 4 + li;
            xr[li][k] = (q < nq && r < a.rows)
                ? reinterpret_cast<const float4 *>(a.xT + r * a.B)[q] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
    uint32_t pos = sd.byte_begin, carry = sd.base_col, ebase = sd.elem_begin;
    const uint32_t end = sd.byte_end;
    while (pos < end) {
        const Chunk ch = decode_chunk(a.idx, pos, end, carry);
        if (ch.T == 0ull) break;
        if (ch.term) {
            s_off[wave][ch.rank] = ch.col * 4u * ld_bytes;
            s_t[wave][ch.rank] = ebase + ch.rank;
        }
        wave_lds_sync();
        const uint32_t n = (uint32_t)__popcll(ch.T);
        for (uint32_t j = 0; j < n; j += G) {
            const uint32_t e = j + g;
            const uint32_t off = e < n ? s_off[wave][e] : OOB_OFFSET;
            float d[16];
#pragma unroll
            for (int lj = 0; lj < 4; ++lj) {
                float4 gv[KB];
#pragma unroll
                for (int k = 0; k < KB; ++k) gv[k] = buffer_load_f4(rg, off + (uint32_t)lj * ld_bytes + lane_off[k]);
#pragma unroll
                for (int li = 0; li < 4; ++li) {
                    // one chain per slot (16 independent chains per lane)
                    float d0 = 0.f;
#pragma unroll
                    for (int k = 0; k < KB; ++k) {
                        d0 = __builtin_fmaf(xr[li][k].x, gv[k].x, d0);
                        d0 = __builtin_fmaf(xr[li][k].y, gv[k].y, d0);
                        d0 = __builtin_fmaf(xr[li][k].z, gv[k].z, d0);
                        d0 = __builtin_fmaf(xr[li][k].w, gv[k].w, d0);
                    }
                    d[lj * 4 + li] = d0;
                }
            }
#pragma unroll
            for (int s = 0; s < 16; ++s) d[s] = group_sum_last<BL>(d[s]);
            if (bl == BL - 1u && e < n) {
                float4 *o = reinterpret_cast<float4 *>(a.gw + (size_t)s_t[wave][e] * 16u);
                o[0] = make_float4(d[0], d[1], d[2], d[3]);
                o[1] = make_float4(d[4], d[5], d[6], d[7]);
                o[2] = make_float4(d[8], d[9], d[10], d[11]);
                o[3] = make_float4(d[12], d[13], d[14], d[15]);
            }
        }
        wave_lds_sync();
        carry = chunk_advance(ch, pos, ebase);
    }
}

// The same sampled grad-W over runs of tiles: run (x, br) = the tiles of
// block row br in column range x (B4Ranges), one wave per run, runs in order
// x-major and the blocks in XCD-contiguous order (xcd_block), so that XCD x
// takes range x's runs: its L2 then holds only that range's gT rows (the
// whole gT of a large layer does not fit one XCD's L2).  The tiles' block
// columns come from tcol (no varint decode).  Per lane the arithmetic and the
// reduction are k_sddmm_b4_v4's, so the results are the same bit for bit.
struct SRArgs {
    const uint32_t *tcol, *start;
    int64_t nruns, brows;
    int64_t rows;
    const float *xT, *gT;
    int64_t B;
    float *gw;
};
template <int BL, int KB>
__global__ __launch_bounds__(256) void k_sddmm_b4_rng(SRArgs a, uint32_t gT_bytes) {
    constexpr uint32_t G = 64u / BL;
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const int64_t run = (int64_t)xcd_block(blockIdx.x, gridDim.x) * WAVES + wave;
    if (run >= a.nruns) return;
    const int64_t br = run % a.brows;
    const uint32_t t0 = a.start[run], t1 = a.start[run + a.brows];
    if (t0 >= t1) return;
    const uint32_t g = lane / BL, bl = lane % BL;
    const uint32_t nq = (uint32_t)(a.B >> 2);
    const uint32_t ld_bytes = (uint32_t)a.B * 4u;
    const __amdgpu_buffer_rsrc_t rg = buffer_rsrc(a.gT, gT_bytes);
    uint32_t lane_off[KB];
    float4 xr[4][KB];
#pragma unroll
    for (int k = 0; k < KB; ++k) {
        const uint32_t q = bl + BL * (uint32_t)k;
        lane_off[k] = q < nq ? q * 16u : OOB_OFFSET;
#pragma unroll
        for (int li = 0; li < 4; ++li) {
            const int64_t r = br * 4 + li;
            xr[li][k] = (q < nq && r < a.rows)
                ? reinterpret_cast<const float4 *>(a.xT + r * a.B)[q] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
    for (uint32_t j = t0; j < t1; j += G) {
        const uint32_t t = j + g;
        const bool ok = t < t1;
        const uint32_t off = ok ? a.tcol[t] * 4u * ld_bytes : OOB_OFFSET;
        float d[16];
#pragma unroll
        for (int lj = 0; lj < 4; ++lj) {
            float4 gv[KB];
#pragma unroll
            for (int k = 0; k < KB; ++k) gv[k] = buffer_load_f4(rg, off + (uint32_t)lj * ld_bytes + lane_off[k]);
#pragma unroll
            for (int li = 0; li < 4; ++li) {
                // one chain per slot (16 independent chains per lane)
                float d0 = 0.f;
#pragma unroll
                for (int k = 0; k < KB; ++k) {
                    d0 = __builtin_fmaf(xr[li][k].x, gv[k].x, d0);
                    d0 = __builtin_fmaf(xr[li][k].y, gv[k].y, d0);
                    d0 = __builtin_fmaf(xr[li][k].z, gv[k].z, d0);
                    d0 = __builtin_fmaf(xr[li][k].w, gv[k].w, d0);
                }
                d[lj * 4 + li] = d0;
            }
        }
#pragma unroll
        for (int s = 0; s < 16; ++s) d[s] = group_sum_last<BL>(d[s]);
        if (bl == BL - 1u && ok) {
            float4 *o = reinterpret_cast<float4 *>(a.gw + (size_t)t * 16u);
            o[0] = make_float4(d[0], d[1], d[2], d[3]);
            o[1] = make_float4(d[4], d[5], d[6], d[7]);
            o[2] = make_float4(d[8], d[9], d[10], d[11]);
            o[3] = make_float4(d[12], d[13], d[14], d[15]);
        }
    }
}

// gw[16*t + lj*4+li] = sum_b xT[4br+li, b] * gT[4bc+lj, b] for every slot.
__global__ __launch_bounds__(256) void k_sddmm_b4(SBArgs a) {
    extern __shared__ __align__(16) float s_x4[];  // [WAVES][4][B]
    __shared__ uint32_t s_bc[WAVES][64];
    __shared__ uint32_t s_t[WAVES][64];
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const int64_t si = (int64_t)blockIdx.x * WAVES + wave;
    if (si >= a.nseg) return;
    const SegDesc sd = a.seg[si];
    const int64_t B = a.B;
    const uint32_t br = sd.row;
    float *sx = s_x4 + (int64_t)wave * 4 * B;
    for (int64_t q = lane; q < 4 * B; q += 64) {
        const int64_t li = q / B, b = q % B;
        const int64_t r = (int64_t)br * 4 + li;
        sx[q] = r < a.rows ? a.xT[r * B + b] : 0.0f;
    }
    uint32_t pos = sd.byte_begin, carry = sd.base_col, ebase = sd.elem_begin;
    const uint32_t end = sd.byte_end;
    const bool vec4 = (B & 3) == 0;
    while (pos < end) {
        const Chunk ch = decode_chunk(a.idx, pos, end, carry);
        if (ch.T == 0ull) break;
        if (ch.term) {
            s_bc[wave][ch.rank] = ch.col;
            s_t[wave][ch.rank] = ebase + ch.rank;
        }
        wave_lds_sync();
        const uint32_t n = (uint32_t)__popcll(ch.T);
        for (uint32_t q = lane; q < n * 16u; q += 64u) {
            const uint32_t jt = q >> 4, slot = q & 15u, li = slot & 3u, lj = slot >> 2;
            const uint32_t c = s_bc[wave][jt] * 4u + lj;
            const uint32_t r = br * 4u + li;
            float acc = 0.0f;
            if (r < a.rows && c < a.cols) {
                const float *gr = a.gT + (int64_t)c * B;
                const float *xr = sx + (int64_t)li * B;
                if (vec4) {
                    acc = dot_f4(xr, gr, B);
                } else {
                    for (int64_t b = 0; b < B; ++b) acc = __builtin_fmaf(xr[b], gr[b], acc);
                }
            }
            a.gw[(size_t)s_t[wave][jt] * 16u + slot] = acc;
        }
        wave_lds_sync();
        carry = chunk_advance(ch, pos, ebase);
    }
}

// [B, n] -> [n, B], one 64(b) x 16(j) tile per block through LDS.  Any
// shape and alignment.  Optional acc[j] += sum_b |x[b,j]| (atomics when B
// spans several tiles).
__global__ __launch_bounds__(256) void k_transpose(const float *__restrict__ src, int64_t B,
                                                   int64_t n, float *__restrict__ dst,
                                                   float *__restrict__ acc) {
    __shared__ float tile[64][17];
    const int64_t j0 = (int64_t)blockIdx.x * 16, b0 = (int64_t)blockIdx.y * 64;
    const uint32_t t = threadIdx.x;
    {
        const uint32_t jj = t & 15u, bb = t >> 4;  // 16 x 16
#pragma unroll
        for (uint32_t i = 0; i < 4u; ++i) {
            const int64_t b = b0 + bb + 16u * i, j = j0 + jj;
            tile[bb + 16u * i][jj] = (b < B && j < n) ? src[b * n + j] : 0.0f;
        }
    }
    __syncthreads();
    if (acc) {
        // 16 lanes per column, 4 rows each
        const uint32_t jj = t >> 4, r = t & 15u;
        float s = 0.0f;
#pragma unroll
        for (uint32_t i = 0; i < 4u; ++i) s += __builtin_fabsf(tile[r * 4u + i][jj]);
        s = group_sum_last<16>(s);
        if (r == 15u && j0 + jj < n) {
            if (gridDim.y == 1) acc[j0 + jj] += s;
            else atomicAdd(acc + j0 + jj, s);
        }
    }
    {
        const uint32_t bb = t & 63u, jj = t >> 6;  // 64 x 4
#pragma unroll
        for (uint32_t i = 0; i < 4u; ++i) {
            const int64_t j = j0 + jj + 4u * i, b = b0 + bb;
            if (j < n && b < B) dst[j * B + b] = tile[bb][jj + 4u * i];
        }
    }
}

// The same with float4 rows: a 64(b) x 32(j) tile, 128-byte reads along j,
// 256-byte writes along b.  Needs n % 4 == 0, B % 4 == 0 and 16-byte aligned
// src / dst.
__device__ __forceinline__ void transpose_v4_body(const float *__restrict__ src, int64_t B, int64_t n,
                                                  float *__restrict__ dst, float *__restrict__ acc, uint32_t bx,
                                                  uint32_t by, uint32_t gy, float (*tile)[33]) {
    const int64_t j0 = (int64_t)bx * 32, b0 = (int64_t)by * 64;
    const uint32_t t = threadIdx.x;
    {
        const uint32_t q = t & 7u, bb = t >> 3;  // 8 float4 per row, 32 rows per pass
#pragma unroll
        for (uint32_t i = 0; i < 2u; ++i) {
            const int64_t b = b0 + bb + 32u * i, j = j0 + 4u * q;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (b < B && j < n) v = *reinterpret_cast<const float4 *>(src + b * n + j);
            float *row = tile[bb + 32u * i];
            row[4u * q] = v.x;
            row[4u * q + 1u] = v.y;
            row[4u * q + 2u] = v.z;
            row[4u * q + 3u] = v.w;
        }
    }
    __syncthreads();
    {
        const uint32_t q = t & 15u, jj = t >> 4;  // 16 float4 per column, 16 columns per pass
#pragma unroll
        for (uint32_t i = 0; i < 2u; ++i) {
            const uint32_t jc = jj + 16u * i;
            const int64_t j = j0 + jc, b = b0 + 4u * q;
            const float4 v = make_float4(tile[4u * q][jc], tile[4u * q + 1u][jc], tile[4u * q + 2u][jc],
                                         tile[4u * q + 3u][jc]);
            if (j < n && b < B) *reinterpret_cast<float4 *>(dst + j * B + b) = v;
            if (acc) {
                float s = (__builtin_fabsf(v.x) + __builtin_fabsf(v.y)) +
                          (__builtin_fabsf(v.z) + __builtin_fabsf(v.w));
                s = group_sum_last<16>(s);
                if (q == 15u && j < n) {
                    if (gy == 1) acc[j] += s;
                    else atomicAdd(acc + j, s);
                }
            }
        }
    }
}
__global__ __launch_bounds__(256) void k_transpose_v4(const float *__restrict__ src, int64_t B,
                                                      int64_t n, float *__restrict__ dst,
                                                      float *__restrict__ acc) {
    __shared__ float tile[64][33];
    transpose_v4_body(src, B, n, dst, acc, blockIdx.x, blockIdx.y, gridDim.y, tile);
}

// acc[j] += sum_b |xT[j*B + b]| over a feature-major copy (one wave per row).
__device__ __forceinline__ void rowabs_body(const float *__restrict__ xT, int64_t B, int64_t n,
                                            float *__restrict__ acc, uint32_t bx) {
    const int64_t j = (int64_t)bx * 4 + (threadIdx.x >> 6);
    if (j >= n) return;
    float s = 0.0f;
    for (int64_t b = threadIdx.x & 63u; b < B; b += 64) s += __builtin_fabsf(xT[j * B + b]);
    s = wave_sum(s);
    if ((threadIdx.x & 63u) == 0) acc[j] += s;
}
__global__ __launch_bounds__(256) void k_rowabs(const float *__restrict__ xT, int64_t B, int64_t n,
                                                float *__restrict__ acc) {
    rowabs_body(xT, B, n, acc, blockIdx.x);
}

__global__ __launch_bounds__(256) void k_colabs(const float *__restrict__ src, int64_t B, int64_t n,
                                                float *__restrict__ acc) {
    const int64_t j = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (j >= n) return;
    float s = 0.0f;
    for (int64_t b = 0; b < B; ++b) s += __builtin_fabsf(src[b * n + j]);
    acc[j] += s;
}

// acc[j] += sum_b |src[b, j]| over a batch-major [B, n] array: 64 columns
// per block as 16 float4 lanes x 16 batch groups, summed through LDS.
// Needs n % 4 == 0 and a 16-byte aligned src.
__device__ __forceinline__ void colabs_v4_body(const float *__restrict__ src, int64_t B, int64_t n,
                                               float *__restrict__ acc, uint32_t bx, float4 (*part)[16]) {
    const uint32_t t = threadIdx.x, q = t & 15u, bg = t >> 4;
    const int64_t j = (int64_t)bx * 64 + 4 * q;
    float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
    if (j < n) {
        for (int64_t b = bg; b < B; b += 16) {
            const float4 v = *reinterpret_cast<const float4 *>(src + b * n + j);
            s.x += __builtin_fabsf(v.x);
            s.y += __builtin_fabsf(v.y);
            s.z += __builtin_fabsf(v.z);
            s.w += __builtin_fabsf(v.w);
        }
    }
    part[bg][q] = s;
    __syncthreads();
    if (bg == 0 && j < n) {
        float4 tot = part[0][q];
        for (int g = 1; g < 16; ++g) {
            const float4 v = part[g][q];
            tot.x += v.x; tot.y += v.y; tot.z += v.z; tot.w += v.w;
        }
        float4 *a4 = reinterpret_cast<float4 *>(acc + j);
        float4 cur = *a4;
        cur.x += tot.x; cur.y += tot.y; cur.z += tot.z; cur.w += tot.w;
        *a4 = cur;
    }
}
__global__ __launch_bounds__(256) void k_colabs_v4(const float *__restrict__ src, int64_t B, int64_t n,
                                                   float *__restrict__ acc) {
    __shared__ float4 part[16][16];
    colabs_v4_body(src, B, n, acc, blockIdx.x, part);
}

// Zero out[b, row] for every row split over several work items (their
// partial sums add atomically); rows with one work item are stored whole.
// One thread per (batch index, split row).
__global__ __launch_bounds__(256) void k_zero_split_rows(const uint32_t *__restrict__ rows, int64_t n_split,
                                                         float *__restrict__ out, int64_t out_ld, int64_t nb) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n_split * nb) return;
    const int64_t b = i / n_split, k = i - b * n_split;
    out[b * out_ld + rows[k]] = 0.0f;
}

__global__ __launch_bounds__(256) void k_zero_f4(float4 *__restrict__ p, int64_t n4) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n4) p[i] = make_float4(0.f, 0.f, 0.f, 0.f);
}
__global__ __launch_bounds__(256) void k_zero_f1(float *__restrict__ p, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) p[i] = 0.0f;
}

// Independent small tasks of one entry point in one launch: each block runs
// the task whose block range holds it (tasks[k].first .. + blocks).
__global__ __launch_bounds__(256) void k_prep(PrepArgs a) {
    __shared__ float tile[64][33];
    uint32_t k = 0;
    while (k + 1 < (uint32_t)a.nt && blockIdx.x >= a.t[k + 1].first) ++k;
    const PrepTask &T = a.t[k];
    const uint32_t vb = blockIdx.x - T.first;
    switch (T.kind) {
    case PREP_TRANSPOSE: {
        const uint32_t gx = (uint32_t)((T.n + 31) / 32), gy = (uint32_t)((T.B + 63) / 64);
        transpose_v4_body(T.src, T.B, T.n, T.dst, T.acc, vb % gx, vb / gx, gy, tile);
        break;
    }
    case PREP_COLABS:
        colabs_v4_body(T.src, T.B, T.n, T.acc, vb, reinterpret_cast<float4 (*)[16]>(&tile[0][0]));
        break;
    case PREP_ROWABS:
        rowabs_body(T.src, T.B, T.n, T.acc, vb);
        break;
    case PREP_FILL4: {
        const int64_t i = (int64_t)vb * 256 + threadIdx.x;
        if (i < T.n) reinterpret_cast<float4 *>(T.dst)[i] = make_float4(T.v, T.v, T.v, T.v);
        break;
    }
    default: {  // PREP_ZERO_LIST: out[b * ld + rows[k]] = 0, n = split rows, B = batch
        const int64_t i = (int64_t)vb * 256 + threadIdx.x;
        if (i < T.n * T.B) {
            const int64_t b = i / T.n, r = i - b * T.n;
            T.dst[b * T.ld + T.rows[r]] = 0.0f;
        }
        break;
    }
    }
}

// CSR activations -> feature-major dst[j, b] (zero-filled beforehand), one
// thread per stored entry; its batch row comes from a binary search of
// ptrs.  Explicit zeros are written as -0.0 when `mark` (so "+0.0 = absent"
// stays distinguishable); optional acc_abs[j] += |v|.
__global__ __launch_bounds__(256) void k_densify_entries(const int32_t *__restrict__ ptrs,
                                                         const int32_t *__restrict__ idx,
                                                         const float *__restrict__ vals, int64_t B, int64_t n,
                                                         float *__restrict__ dst, float *__restrict__ acc_abs,
                                                         int mark) {
    const int64_t p = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t total = ptrs[B];
    if (p >= total) return;
    int64_t lo = 0, hi = B;  // last b with ptrs[b] <= p
    while (hi - lo > 1) {
        const int64_t mid = (lo + hi) >> 1;
        if (ptrs[mid] <= p) lo = mid;
        else hi = mid;
    }
    const int64_t j = idx[p];
    if (j < 0 || j >= n) return;  // host validated; never write out of bounds
    float v = vals[p];
    if (acc_abs) atomicAdd(acc_abs + j, __builtin_fabsf(v));
    if (mark && __builtin_bit_cast(uint32_t, v) == 0u) v = -0.0f;
    dst[j * B + lo] = v;
}

// CSR activations (indices ascending within a batch row) -> the whole
// feature-major dst[j * B + b], zeros where absent: one block per tile of R
// rows, built in LDS and written out whole -- the zero fill and the scatter
// in one pass.  Each batch row's first and last entries in the tile are
// found at once by a group of G lanes each (a G-ary search: every round the
// group samples G evenly spaced indices and keeps the bracket that holds
// the key, so a row of len entries takes log_G(len) dependent loads); a
// block scan places the entries and all of them are loaded in one round.
// Explicit zeros become -0.0 when `mark`; acc_abs[j] += |v| (optional).
// 2 * B * G <= 1024, G in [2, 32], B <= DENSIFY_TILE_MAX_B.
constexpr int64_t DENSIFY_TILE_MAX_B = 256;
__global__ __launch_bounds__(1024) void k_densify_tiles(const int32_t *__restrict__ ptrs,
                                                        const int32_t *__restrict__ idx,
                                                        const float *__restrict__ vals, int64_t B, int64_t n,
                                                        int64_t R, uint32_t lg, float *__restrict__ dst,
                                                        float *__restrict__ acc_abs, int mark) {
    extern __shared__ float tile[];  // R * B floats
    __shared__ int32_t s_lo[DENSIFY_TILE_MAX_B], s_hi[DENSIFY_TILE_MAX_B];
    __shared__ uint32_t s_pre[DENSIFY_TILE_MAX_B + 1];
    __shared__ uint32_t s_wave[16];
    const int64_t j0 = (int64_t)blockIdx.x * R;
    const int64_t rows = min<int64_t>(R, n - j0), cnt = rows * B;
    const uint32_t t = threadIdx.x, lane = t & 63u, wave = t >> 6;
    for (int64_t i = t; i < cnt; i += 1024) tile[i] = 0.0f;
    const uint32_t G = 1u << lg, q = t >> lg, k = t & (G - 1u);
    if ((int64_t)q < 2 * B) {
        const int64_t b = q >> 1, key = j0 + ((q & 1u) ? rows : 0);
        int64_t lo = ptrs[b], hi = ptrs[b + 1];  // the answer lies in [lo, hi]
        const uint64_t gmask = (((uint64_t)1 << G) - 1u) << (lane & ~(G - 1u));
        while (lo < hi) {
            const int64_t step = (hi - lo + G - 1) >> lg;
            const int64_t pos = lo + (int64_t)k * step;
            const bool below = pos < hi && idx[pos] < key;
            const int64_t c = __popcll(__ballot(below) & gmask);
            if (c == 0) {
                hi = lo;
            } else {
                hi = min<int64_t>(hi, lo + c * step);
                lo = lo + (c - 1) * step + 1;
            }
        }
        if (k == 0) ((q & 1u) ? s_hi : s_lo)[b] = (int32_t)lo;
    }
    __syncthreads();
    const uint32_t c = (int64_t)t < B ? (uint32_t)(s_hi[t] - s_lo[t]) : 0u;
    // exclusive scan of the counts over the batch rows
    uint32_t incl = c;
    for (uint32_t o = 1; o < 64u; o <<= 1) {
        const uint32_t y = __shfl_up(incl, o, 64);
        if (lane >= o) incl += y;
    }
    if (lane == 63u) s_wave[wave] = incl;
    __syncthreads();
    uint32_t before = 0, total = 0;
    for (uint32_t w = 0; w < 16u; ++w) {
        const uint32_t v = s_wave[w];
        before += w < wave ? v : 0u;
        total += v;
    }
    if ((int64_t)t < B) s_pre[t] = before + incl - c;
    if (t == 0) s_pre[B] = total;
    __syncthreads();
    for (uint32_t e = t; e < total; e += 1024) {
        uint32_t lo = 0, hi = (uint32_t)B;  // last b with s_pre[b] <= e
        while (hi - lo > 1) {
            const uint32_t mid = (lo + hi) >> 1;
            if (s_pre[mid] <= e) lo = mid;
            else hi = mid;
        }
        const int64_t p = s_lo[lo] + (int64_t)(e - s_pre[lo]);
        const int64_t j = idx[p];
        if (j < j0 || j >= j0 + rows) continue;  // never written out of its tile
        float v = vals[p];
        if (acc_abs) atomicAdd(acc_abs + j, __builtin_fabsf(v));
        if (mark && __builtin_bit_cast(uint32_t, v) == 0u) v = -0.0f;
        tile[(j - j0) * B + lo] = v;
    }
    __syncthreads();
    float *out = dst + j0 * B;
    if ((reinterpret_cast<uintptr_t>(out) & 15u) == 0 && (cnt & 3) == 0) {
        for (int64_t i = t; i < cnt / 4; i += 1024)
            reinterpret_cast<float4 *>(out)[i] = reinterpret_cast<const float4 *>(tile)[i];
    } else {
        for (int64_t i = t; i < cnt; i += 1024) out[i] = tile[i];
    }
}

struct DArgs {
    const SegDesc *seg;
    int64_t nseg;
    const uint8_t *idx;
    const uint8_t *val;
    ScaleView sc;
    int32_t *cols;
    float *w;
    uint32_t *rows_out;
};

__global__ __launch_bounds__(256) void k_decode(DArgs a) {
    const uint32_t wave = threadIdx.x >> 6;
    __shared__ SegStage s_stage[WAVES];
    const int64_t si = (int64_t)blockIdx.x * WAVES + wave;
    if (si >= a.nseg) return;
    const SegDesc sd = a.seg[si];
    const StagedSeg sg = stage_segment(s_stage[wave], a.idx, a.val, sd);
    uint32_t pos = 0, carry = sd.base_col, ebase = sd.elem_begin;
    const uint32_t end = sg.end;
    while (pos < end) {
        const Chunk ch = decode_chunk(sg.idx, pos, end, carry);
        if (ch.T == 0ull) break;
        if (ch.term) {
            const uint32_t e = ebase + ch.rank;
            if (a.cols) a.cols[e] = (int32_t)ch.col;
            if (a.w) a.w[e] = fp4_decode((uint32_t)sg.val[e - sd.elem_begin] >> 4) * scale_at(a.sc, sd.row, ch.col);
            if (a.rows_out) a.rows_out[e] = sd.row;
        }
        carry = chunk_advance(ch, pos, ebase);
    }
}

__global__ __launch_bounds__(256) void k_decode_b4(const SegDesc *seg, int64_t nseg,
                                                   const uint8_t *idx, uint32_t *tile_br,
                                                   uint32_t *tile_bc) {
    const uint32_t wave = threadIdx.x >> 6;
    const int64_t si = (int64_t)blockIdx.x * WAVES + wave;
    if (si >= nseg) return;
    const SegDesc sd = seg[si];
    uint32_t pos = sd.byte_begin, carry = sd.base_col, ebase = sd.elem_begin;
    const uint32_t end = sd.byte_end;
    while (pos < end) {
        const Chunk ch = decode_chunk(idx, pos, end, carry);
        if (ch.T == 0ull) break;
        if (ch.term) {
            const uint32_t t = ebase + ch.rank;
            if (tile_br) tile_br[t] = sd.row;
            if (tile_bc) tile_bc[t] = ch.col;
        }
        carry = chunk_advance(ch, pos, ebase);
    }
}

inline unsigned blocks_for(int64_t nseg) { return (unsigned)((nseg + WAVES - 1) / WAVES); }

template <int G, int KB>
void gather_dispatch_skip(const GArgs &a, int skip, hipStream_t st) {
    const dim3 grid(blocks_for(a.nseg)), block(256);
    switch (skip) {
        case SKIP_ZERO: launch((k_gather<G, KB, SKIP_ZERO>), grid, block, 0, st, a); break;
        case SKIP_POSZERO: launch((k_gather<G, KB, SKIP_POSZERO>), grid, block, 0, st, a); break;
        default: launch((k_gather<G, KB, SKIP_NONE>), grid, block, 0, st, a); break;
    }
}

template <int G, int KB>
void gather_b4_dispatch_skip(const BArgs &a, int skip, hipStream_t st) {
    const dim3 grid(blocks_for(a.nseg)), block(256);
    switch (skip) {
        case SKIP_ZERO: launch((k_gather_b4<G, KB, SKIP_ZERO>), grid, block, 0, st, a); break;
        case SKIP_POSZERO: launch((k_gather_b4<G, KB, SKIP_POSZERO>), grid, block, 0, st, a); break;
        default: launch((k_gather_b4<G, KB, SKIP_NONE>), grid, block, 0, st, a); break;
    }
}

template <int BL, int KB, int U>
void gather_v4_skip_u(const GArgs &a, int skip, hipStream_t st) {
    // with short rows: the long work items' blocks, then the short rows' blocks
    const dim3 grid(a.sh_seg ? a.n_lgblk + blocks_for((a.n_sh + SHORT_R_MAX - 1) / SHORT_R_MAX)
                             : blocks_for(a.nseg)),
        block(256);
    switch (skip) {
        case SKIP_ZERO: launch((k_gather_v4<BL, KB, U, SKIP_ZERO>), grid, block, 0, st, a); break;
        case SKIP_POSZERO: launch((k_gather_v4<BL, KB, U, SKIP_POSZERO>), grid, block, 0, st, a); break;
        default: launch((k_gather_v4<BL, KB, U, SKIP_NONE>), grid, block, 0, st, a); break;
    }
}

// Launch-shape knobs of the float4 kernels (environment, read once):
//   SILI_GATHER_BL  lanes per entry at batch 64 / 128 (4, 8 or 16)
//   SILI_GATHER_U   entries per lane group in flight
// Defaults: 8 lanes per entry (G = 8 entries per load instruction, two
// float4 chunks per lane at batch 64); 4 entries per group in flight in the
// gathers and 2 in the fused backward, the shapes that keep 8 waves per
// SIMD (64 VGPRs, 20 KiB of LDS per block of 4 waves): config 1's 8192
// work items then run in one round of resident waves.
inline int gather_bl() {
    static const int v = [] {
        const int b = env_int("SILI_GATHER_BL", 8);
        return b >= 16 ? 16 : b >= 8 ? 8 : 4;
    }();
    return v;
}
inline int gather_u() {
    static const int v = env_int("SILI_GATHER_U", 0);  // 0: per-shape default
    return v;
}

template <int BL, int KB>
void gather_v4_skip(const GArgs &a, int skip, hipStream_t st) {
    const int u = gather_u();
    if constexpr (KB >= 4) {
        if (u >= 4) gather_v4_skip_u<BL, KB, 4>(a, skip, st);
        else if (u >= 2) gather_v4_skip_u<BL, KB, 2>(a, skip, st);
        else gather_v4_skip_u<BL, KB, 1>(a, skip, st);
    } else {
        if (u >= 16 && KB == 1) gather_v4_skip_u<BL, KB, 16>(a, skip, st);
        else if (u >= 8) gather_v4_skip_u<BL, KB, 8>(a, skip, st);
        else gather_v4_skip_u<BL, KB, 4>(a, skip, st);
    }
}

inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// SILI_XCD_ORDER (read per call): 1 the float4 segment kernels take their
// blocks in XCD-contiguous order (xcd_block), 0 in launch order.  Default:
// on for the fused backward (c1: 26.2 -> 25.7 us), off for the gathers
// (no gain at batch 64; c4's batch-128 gathers lose 14%).
inline int xcd_order(int dflt) { return env_int("SILI_XCD_ORDER", dflt) ? 1 : 0; }

}  // namespace

void launch_gather(const GatherPlan &p, const ScaleView &sc, const float *in, int64_t in_ld,
                   float *out, int64_t out_ld, int64_t nb_total, int skip, hipStream_t st, bool accumulate) {
    if (p.nseg == 0 || nb_total == 0) return;
    ProfScope ps("gather", st);
    for (int64_t b0 = 0; b0 < nb_total; b0 += 512) {
        const int64_t nb = nb_total - b0 < 512 ? nb_total - b0 : 512;
        const int64_t in_bytes = (p.cols * in_ld - b0) * 4;
        const bool small = in_bytes < (int64_t)OOB_OFFSET;
        GArgs a{p.seg, p.nseg, p.idx, p.val, sc, in + b0, in_ld, out + b0 * out_ld, out_ld, nb,
                small ? (uint32_t)in_bytes : 0u, accumulate ? 1 : 0, xcd_order(0), nullptr, nullptr, nullptr};
        if (accumulate && !(small && nb % 4 == 0 && in_ld % 4 == 0 && aligned16(a.in)))
            throw_error(3, "launch_gather: accumulating passes need the float4 kernels");
        const bool v4 = small && nb % 4 == 0 && in_ld % 4 == 0 && aligned16(a.in);
        if (v4 && p.has_split && p.part && p.nseg * nb <= p.part_cap) {
            a.elem_start = p.elem_start;
            a.split_cnt = p.split_cnt;
            a.part = p.part;
        }
        // short rows several to a wave (the shapes up to SHORT_MAX_BATCH
        // columns; the dispatch below picks one of them for nb <= 64)
        if (v4 && p.sh_seg && p.n_sh > 0 && nb > 1 && nb <= SHORT_MAX_BATCH) {
            a.seg = p.lg_seg;
            a.nseg = p.n_lg;
            a.sh_seg = p.sh_seg;
            a.n_sh = p.n_sh;
            a.n_lgblk = blocks_for(p.n_lg);
        }

        const dim3 grid(blocks_for(a.nseg)), block(256);
        if (nb == 1 && small) {
            static const int lane_decode = env_int("SILI_B1_LANE_DECODE", 2);
            // (static LDS ~12.8 KB + the input stay within 64 KB per block)
            // (only when each resident block has many segments to amortize the copy over)
            if (lane_decode == 2 && skip == SKIP_NONE && sc.rank == 1 && in_ld == 1 && p.cols * 4 + 13312 <= 65536 &&
                p.nseg >= (int64_t)256 * 4 * WAVES * 8) {
                // input (times its column scale) held in LDS by each persistent block
                const size_t lds = (size_t)p.cols * 4;
                const unsigned gp = (unsigned)std::min<int64_t>((int64_t)blocks_for(a.nseg), 256 * (lds <= 24576 ? 4 : 2));
                launch(k_gather_b1p<SKIP_NONE, true, true>, dim3(gp), block, (uint32_t)lds, st, a, 0u);
                SILI_HIP(hipGetLastError());
                continue;
            }
            if (lane_decode == 2 && p.cols < (1 << 28)) {
                // persistent pipelined waves: enough to fill the chip, no more
                const unsigned gp = (unsigned)std::min<int64_t>((int64_t)blocks_for(a.nseg), 256 * 6);
                const uint32_t eb2 = (uint32_t)(p.cols * 4 < (int64_t)OOB_OFFSET ? p.cols * 4 : 0);
                switch ((skip == SKIP_ZERO ? 0 : skip == SKIP_POSZERO ? 1 : 2) + (sc.rank == 1 ? 0 : 3)) {
                    case 0: launch(k_gather_b1p<SKIP_ZERO, true>, dim3(gp), block, 0, st, a, eb2); break;
                    case 1: launch(k_gather_b1p<SKIP_POSZERO, true>, dim3(gp), block, 0, st, a, eb2); break;
                    case 2: launch(k_gather_b1p<SKIP_NONE, true>, dim3(gp), block, 0, st, a, eb2); break;
                    case 3: launch(k_gather_b1p<SKIP_ZERO, false>, dim3(gp), block, 0, st, a, eb2); break;
                    case 4: launch(k_gather_b1p<SKIP_POSZERO, false>, dim3(gp), block, 0, st, a, eb2); break;
                    default: launch(k_gather_b1p<SKIP_NONE, false>, dim3(gp), block, 0, st, a, eb2); break;
                }
                SILI_HIP(hipGetLastError());
                continue;
            }
            const uint32_t eb = (uint32_t)(p.cols * 4 < (int64_t)OOB_OFFSET ? p.cols * 4 : 0);
            if (lane_decode && sc.rank == 1) {
                switch (skip) {
                    case SKIP_ZERO: launch(k_gather_b1s<SKIP_ZERO, true>, grid, block, 0, st, a, eb); break;
                    case SKIP_POSZERO: launch(k_gather_b1s<SKIP_POSZERO, true>, grid, block, 0, st, a, eb); break;
                    default: launch(k_gather_b1s<SKIP_NONE, true>, grid, block, 0, st, a, eb); break;
                }
            } else if (lane_decode) {
                switch (skip) {
                    case SKIP_ZERO: launch(k_gather_b1s<SKIP_ZERO, false>, grid, block, 0, st, a, eb); break;
                    case SKIP_POSZERO: launch(k_gather_b1s<SKIP_POSZERO, false>, grid, block, 0, st, a, eb); break;
                    default: launch(k_gather_b1s<SKIP_NONE, false>, grid, block, 0, st, a, eb); break;
                }
            } else {
                switch (skip) {
                    case SKIP_ZERO: launch(k_gather_b1<SKIP_ZERO>, grid, block, 0, st, a); break;
                    case SKIP_POSZERO: launch(k_gather_b1<SKIP_POSZERO>, grid, block, 0, st, a); break;
                    default: launch(k_gather_b1<SKIP_NONE>, grid, block, 0, st, a); break;
                }
            }
        } else if (v4) {
            const int64_t nq = nb / 4;
            if (nq <= 1) gather_v4_skip<1, 1>(a, skip, st);
            else if (nq <= 2) gather_v4_skip<2, 1>(a, skip, st);
            else if (nq <= 4) gather_v4_skip<4, 1>(a, skip, st);
            else if (nq <= 8) gather_v4_skip<8, 1>(a, skip, st);
            else if (nq <= 16) {
                const int bl = gather_bl();
                if (nq > 8 && bl == 4) gather_v4_skip<4, 4>(a, skip, st);
                else if (nq > 8 && bl == 8) gather_v4_skip<8, 2>(a, skip, st);
                else gather_v4_skip<16, 1>(a, skip, st);
            } else if (nq <= 32) {
                const int bl = gather_bl();
                if (bl == 4) gather_v4_skip<4, 8>(a, skip, st);
                else if (bl == 8) gather_v4_skip<8, 4>(a, skip, st);
                else gather_v4_skip<16, 2>(a, skip, st);
            }
            else if (nq <= 64) gather_v4_skip<16, 4>(a, skip, st);
            else gather_v4_skip<16, 8>(a, skip, st);
        } else if (nb <= 1) gather_dispatch_skip<64, 1>(a, skip, st);
        else if (nb <= 2) gather_dispatch_skip<32, 1>(a, skip, st);
        else if (nb <= 4) gather_dispatch_skip<16, 1>(a, skip, st);
        else if (nb <= 8) gather_dispatch_skip<8, 1>(a, skip, st);
        else if (nb <= 16) gather_dispatch_skip<4, 1>(a, skip, st);
        else if (nb <= 32) gather_dispatch_skip<2, 1>(a, skip, st);
        else if (nb <= 64) gather_dispatch_skip<1, 1>(a, skip, st);
        else if (nb <= 128) gather_dispatch_skip<1, 2>(a, skip, st);
        else if (nb <= 256) gather_dispatch_skip<1, 4>(a, skip, st);
        else gather_dispatch_skip<1, 8>(a, skip, st);
        SILI_HIP(hipGetLastError());
    }
}

void launch_gather_b4(const Block4Plan &p, const ScaleView &sc, const float *in, int64_t in_ld,
                      float *out, int64_t out_ld, int64_t nb_total, int skip, hipStream_t st) {
    if (p.nseg == 0 || nb_total == 0) return;
    ProfScope ps("gather_b4", st);
    const int64_t in_bytes = p.cols * in_ld * 4;
    if (skip == SKIP_NONE && nb_total % 4 == 0 && in_ld % 4 == 0 && aligned16(in) &&
        in_bytes < (int64_t)OOB_OFFSET) {
        BArgs a{p.seg, p.nseg, p.idx, p.tiles, p.rows, p.cols, sc, in, in_ld, out, out_ld, nb_total};
        const int64_t nq = nb_total / 4;
        const unsigned gx = blocks_for(p.nseg);
        const unsigned gy16 = (unsigned)((nq + 15) / 16);
        const int use_mfma = env_int("SILI_B4_MFMA", 0);  // (knobs read per call)
        if (use_mfma && nq >= 12) {
            // matrix cores: 64 batch columns per wave (SILI_B4_MFMA=0: vector path)
            const int u = env_int("SILI_B4_MFMA_U", 2);
            if (u >= 4) launch((k_gather_b4_mfma<4>), dim3(gx, gy16), dim3(256), 0, st, a, (uint32_t)in_bytes);
            else if (u >= 2) launch((k_gather_b4_mfma<2>), dim3(gx, gy16), dim3(256), 0, st, a, (uint32_t)in_bytes);
            else launch((k_gather_b4_mfma<1>), dim3(gx, gy16), dim3(256), 0, st, a, (uint32_t)in_bytes);
        } else if (nq <= 4) {
            launch((k_gather_b4_v4<4, 1, 2>), dim3(gx, 1), dim3(256), 0, st, a, (uint32_t)in_bytes);
        } else if (nq <= 8) {
            launch((k_gather_b4_v4<8, 1, 2>), dim3(gx, 1), dim3(256), 0, st, a, (uint32_t)in_bytes);
        } else {
            // 64 batch columns per wave; lanes per tile and tiles in flight
            // (SILI_B4_BL / SILI_B4_U)
            const int bl = env_int("SILI_B4_BL", 16), u = env_int("SILI_B4_U", 2);
            const unsigned gy8 = (unsigned)((nq + 7) / 8);
            // batches of 128 and more: 128 columns per wave (32 lanes per
            // tile, 2 tile groups in flight), so each tile is decoded and
            // dequantised by half as many waves (SILI_B4_WIDE)
            if (nq >= 32 && bl == 16 && u == 2 && env_int("SILI_B4_WIDE", 1)) {
                const unsigned gyw = (unsigned)((nq + 31) / 32);
                if (env_int("SILI_B4_XCDQ", 1) && gyw > 1) a.xq_gx = gx;
                const dim3 gw = a.xq_gx ? dim3(gx * gyw) : dim3(gx, gyw);
                launch((k_gather_b4_v4<32, 1, 2>), gw, dim3(256), 0, st, a, (uint32_t)in_bytes);
                SILI_HIP(hipGetLastError());
                return;
            }
            // batch chunks on their own XCDs (SILI_B4_XCDQ)
            if (env_int("SILI_B4_XCDQ", 1) && bl == 16 && gy16 > 1) {
                a.xq_gx = gx;
                const dim3 g1(gx * gy16);
                if (u >= 4) launch((k_gather_b4_v4<16, 1, 4>), g1, dim3(256), 0, st, a, (uint32_t)in_bytes);
                else if (u >= 2) launch((k_gather_b4_v4<16, 1, 2>), g1, dim3(256), 0, st, a, (uint32_t)in_bytes);
                else launch((k_gather_b4_v4<16, 1, 1>), g1, dim3(256), 0, st, a, (uint32_t)in_bytes);
                SILI_HIP(hipGetLastError());
                return;
            }
            if (bl == 32 && u >= 4) launch((k_gather_b4_v4<8, 1, 4>), dim3(gx, gy8), dim3(256), 0, st, a, (uint32_t)in_bytes);
            else if (bl == 32) launch((k_gather_b4_v4<8, 1, 2>), dim3(gx, gy8), dim3(256), 0, st, a, (uint32_t)in_bytes);
            else if (bl == 64 && u >= 8) launch((k_gather_b4_w<8>), dim3(gx, gy16), dim3(256), 0, st, a, (uint32_t)in_bytes);
            else if (bl == 64 && u >= 4) launch((k_gather_b4_w<4>), dim3(gx, gy16), dim3(256), 0, st, a, (uint32_t)in_bytes);
            else if (bl == 64) launch((k_gather_b4_w<2>), dim3(gx, gy16), dim3(256), 0, st, a, (uint32_t)in_bytes);
            else if (bl == 8 && u >= 4) launch((k_gather_b4_v4<8, 2, 4>), dim3(gx, gy16), dim3(256), 0, st, a, (uint32_t)in_bytes);
            else if (bl == 8 && u >= 2) launch((k_gather_b4_v4<8, 2, 2>), dim3(gx, gy16), dim3(256), 0, st, a, (uint32_t)in_bytes);
            else if (bl == 8) launch((k_gather_b4_v4<8, 2, 1>), dim3(gx, gy16), dim3(256), 0, st, a, (uint32_t)in_bytes);
            else if (u >= 4) launch((k_gather_b4_v4<16, 1, 4>), dim3(gx, gy16), dim3(256), 0, st, a, (uint32_t)in_bytes);
            else if (u >= 2) launch((k_gather_b4_v4<16, 1, 2>), dim3(gx, gy16), dim3(256), 0, st, a, (uint32_t)in_bytes);
            else launch((k_gather_b4_v4<16, 1, 1>), dim3(gx, gy16), dim3(256), 0, st, a, (uint32_t)in_bytes);
        }
        SILI_HIP(hipGetLastError());
        return;
    }
    for (int64_t b0 = 0; b0 < nb_total; b0 += 256) {
        const int64_t nb = nb_total - b0 < 256 ? nb_total - b0 : 256;
        BArgs a{p.seg, p.nseg, p.idx, p.tiles, p.rows, p.cols, sc, in + b0, in_ld,
                out + b0 * out_ld, out_ld, nb};
        if (nb == 1) gather_b4_dispatch_skip<64, 1>(a, skip, st);
        else if (nb <= 2) gather_b4_dispatch_skip<32, 1>(a, skip, st);
        else if (nb <= 4) gather_b4_dispatch_skip<16, 1>(a, skip, st);
        else if (nb <= 8) gather_b4_dispatch_skip<8, 1>(a, skip, st);
        else if (nb <= 16) gather_b4_dispatch_skip<4, 1>(a, skip, st);
        else if (nb <= 32) gather_b4_dispatch_skip<2, 1>(a, skip, st);
        else if (nb <= 64) gather_b4_dispatch_skip<1, 1>(a, skip, st);
        else if (nb <= 128) gather_b4_dispatch_skip<1, 2>(a, skip, st);
        else gather_b4_dispatch_skip<1, 4>(a, skip, st);
        SILI_HIP(hipGetLastError());
    }
}

void launch_sddmm(const GatherPlan &p, const float *xT, const float *gT, int64_t B, float *gw,
                  float *acc_in, hipStream_t st) {
    if (p.nseg == 0) return;
    ProfScope ps("sddmm", st);
    const int64_t gT_bytes = p.cols * B * 4;
    SArgs a{p.seg, p.nseg, p.idx, xT, gT, B, gw, acc_in,
            gT_bytes < (int64_t)OOB_OFFSET ? (uint32_t)gT_bytes : 0u};
    const dim3 grid(blocks_for(p.nseg)), block(256);
    if (gT_bytes < (int64_t)OOB_OFFSET && B % 4 == 0 && B <= 2048 && aligned16(xT) && aligned16(gT)) {
        const int64_t nq = B / 4;
        const int u = gather_u();
        if (nq <= 1) launch((k_sddmm_v4<1, 1, 1>), grid, block, 0, st, a);
        else if (nq <= 2) launch((k_sddmm_v4<2, 1, 2>), grid, block, 0, st, a);
        else if (nq <= 4) launch((k_sddmm_v4<4, 1, 4>), grid, block, 0, st, a);
        else if (nq <= 8) launch((k_sddmm_v4<8, 1, 8>), grid, block, 0, st, a);
        else if (nq <= 16) {
            if (u >= 16) launch((k_sddmm_v4<16, 1, 16>), grid, block, 0, st, a);
            else if (u >= 8) launch((k_sddmm_v4<16, 1, 8>), grid, block, 0, st, a);
            else launch((k_sddmm_v4<16, 1, 4>), grid, block, 0, st, a);
        } else if (nq <= 32) launch((k_sddmm_v4<16, 2, 4>), grid, block, 0, st, a);
        else if (nq <= 64) launch((k_sddmm_v4<16, 4, 2>), grid, block, 0, st, a);
        else if (nq <= 128) launch((k_sddmm_v4<16, 8, 1>), grid, block, 0, st, a);
        else if (nq <= 256) launch((k_sddmm_v4<16, 16, 1>), grid, block, 0, st, a);
        else launch((k_sddmm_v4<16, 32, 1>), grid, block, 0, st, a);
    } else {
        const size_t lds = sizeof(float) * (size_t)WAVES * (size_t)B;
        if (lds > 64 * 1024) throw_error(1, "sampled grad-W: batch too large for one launch (max 4096)");
        launch(k_sddmm, grid, block, lds, st, a);
    }
    SILI_HIP(hipGetLastError());
}

bool launch_bwd_fused(const GatherPlan &p, const ScaleView &sc, const float *gT, const float *xT,
                      int64_t B, float *dx, int64_t dx_ld, float *gw, float *acc_in, hipStream_t st) {
    const int64_t gT_bytes = p.cols * B * 4;
    if (B % 4 != 0 || B > 512 || gT_bytes >= (int64_t)OOB_OFFSET || !aligned16(xT) || !aligned16(gT))
        return false;
    if (p.nseg == 0) return true;
    ProfScope ps("gather_gradw", st);
    FArgs a{p.seg, p.nseg, p.idx, p.val, sc, gT, (uint32_t)gT_bytes, xT, B, dx, dx_ld, gw, acc_in,
            xcd_order(1), nullptr, nullptr, nullptr};
    if (p.has_split && p.part && p.nseg * B <= p.part_cap) {
        a.elem_start = p.elem_start;
        a.split_cnt = p.split_cnt;
        a.part = p.part;
    }
    const dim3 grid(blocks_for(p.nseg)), block(256);
    const int64_t nq = B / 4;
    if (nq <= 1) launch((k_bwd_v4<1, 1, 4>), grid, block, 0, st, a);
    else if (nq <= 2) launch((k_bwd_v4<2, 1, 4>), grid, block, 0, st, a);
    else if (nq <= 4) launch((k_bwd_v4<4, 1, 4>), grid, block, 0, st, a);
    else if (nq <= 8) launch((k_bwd_v4<8, 1, 4>), grid, block, 0, st, a);
    else if (nq <= 16) {
        const int bl = gather_bl(), u = gather_u();
        if (nq > 8 && bl == 4) {
            if (u >= 2) launch((k_bwd_v4<4, 4, 2>), grid, block, 0, st, a);
            else launch((k_bwd_v4<4, 4, 1>), grid, block, 0, st, a);
        } else if (nq > 8 && bl == 8) {
            // 2 entries per group in flight: 60 VGPRs, so 8 waves per SIMD
            // (4 in flight: 80 VGPRs, 6 waves; 22.6 against 26.1 us on the
            // config-1 grad-input + grad-W)
            if (u >= 4) launch((k_bwd_v4<8, 2, 4>), grid, block, 0, st, a);
            else launch((k_bwd_v4<8, 2, 2>), grid, block, 0, st, a);
        } else launch((k_bwd_v4<16, 1, 4>), grid, block, 0, st, a);
    } else if (nq <= 32) {
        const int bl = gather_bl();
        if (bl == 4) launch((k_bwd_v4<4, 8, 1>), grid, block, 0, st, a);
        else if (bl == 8) launch((k_bwd_v4<8, 4, 1>), grid, block, 0, st, a);
        else launch((k_bwd_v4<16, 2, 4>), grid, block, 0, st, a);
    }
    else if (nq <= 64) launch((k_bwd_v4<16, 4, 2>), grid, block, 0, st, a);
    else launch((k_bwd_v4<16, 8, 1>), grid, block, 0, st, a);
    SILI_HIP(hipGetLastError());
    return true;
}

void launch_sddmm_b4(const Block4Plan &p, const B4Ranges *rng, const float *xT, const float *gT,
                     int64_t B, float *gw, hipStream_t st) {
    if (p.nseg == 0) return;
    ProfScope ps("sddmm_b4", st);
    SBArgs a{p.seg, p.nseg, p.idx, p.rows, p.cols, xT, gT, B, gw};
    const int64_t gT_bytes = p.cols * B * 4;
    if (B % 4 == 0 && B <= 256 && gT_bytes < (int64_t)OOB_OFFSET && aligned16(xT) && aligned16(gT) &&
        aligned16(gw)) {
        const dim3 grid(blocks_for(p.nseg)), block(256);
        const int64_t nq = B / 4;
        if (rng && rng->K >= 1 && rng->tcol && rng->start) {
            const int64_t nruns = rng->K * rng->brows;
            SRArgs r{rng->tcol, rng->start, nruns, rng->brows, p.rows, xT, gT, B, gw};
            const dim3 rgrid(blocks_for(nruns));
            if (nq <= 4) launch((k_sddmm_b4_rng<4, 1>), rgrid, block, 0, st, r, (uint32_t)gT_bytes);
            else if (nq <= 8) launch((k_sddmm_b4_rng<8, 1>), rgrid, block, 0, st, r, (uint32_t)gT_bytes);
            else if (nq <= 16) launch((k_sddmm_b4_rng<16, 1>), rgrid, block, 0, st, r, (uint32_t)gT_bytes);
            else if (nq <= 32) launch((k_sddmm_b4_rng<16, 2>), rgrid, block, 0, st, r, (uint32_t)gT_bytes);
            else launch((k_sddmm_b4_rng<16, 4>), rgrid, block, 0, st, r, (uint32_t)gT_bytes);
            SILI_HIP(hipGetLastError());
            return;
        }
        const int use_mfma = env_int("SILI_B4_MFMA", 0);  // (knobs read per call)
        if (use_mfma && nq >= 8) {
            if (nq <= 16) launch((k_sddmm_b4_mfma<1, 2>), grid, block, 0, st, a, (uint32_t)gT_bytes);
            else if (nq <= 32) launch((k_sddmm_b4_mfma<2, 2>), grid, block, 0, st, a, (uint32_t)gT_bytes);
            else launch((k_sddmm_b4_mfma<4, 2>), grid, block, 0, st, a, (uint32_t)gT_bytes);
        } else if (nq <= 4) launch((k_sddmm_b4_v4<4, 1>), grid, block, 0, st, a, (uint32_t)gT_bytes);
        else if (nq <= 8) launch((k_sddmm_b4_v4<8, 1>), grid, block, 0, st, a, (uint32_t)gT_bytes);
        else if (nq <= 16) launch((k_sddmm_b4_v4<16, 1>), grid, block, 0, st, a, (uint32_t)gT_bytes);
        else if (nq <= 32) launch((k_sddmm_b4_v4<16, 2>), grid, block, 0, st, a, (uint32_t)gT_bytes);
        else launch((k_sddmm_b4_v4<16, 4>), grid, block, 0, st, a, (uint32_t)gT_bytes);
        SILI_HIP(hipGetLastError());
        return;
    }
    const size_t lds = sizeof(float) * (size_t)WAVES * 4u * (size_t)B;
    if (lds > 64 * 1024) throw_error(1, "block4 sampled grad-W: batch too large (max 1024)");
    launch(k_sddmm_b4, dim3(blocks_for(p.nseg)), dim3(256), lds, st, a);
    SILI_HIP(hipGetLastError());
}

void launch_transpose(const float *src, int64_t B, int64_t n, float *dst, float *acc,
                      hipStream_t st) {
    if (B == 0 || n == 0) return;
    ProfScope ps("transpose", st);
    if (n % 4 == 0 && B % 4 == 0 && aligned16(src) && aligned16(dst)) {
        const dim3 grid((unsigned)((n + 31) / 32), (unsigned)((B + 63) / 64));
        launch(k_transpose_v4, grid, dim3(256), 0, st, src, B, n, dst, acc);
    } else {
        const dim3 grid((unsigned)((n + 15) / 16), (unsigned)((B + 63) / 64));
        launch(k_transpose, grid, dim3(256), 0, st, src, B, n, dst, acc);
    }
    SILI_HIP(hipGetLastError());
}

uint32_t prep_blocks(const PrepTask &t) {
    switch (t.kind) {
    case PREP_TRANSPOSE: return (uint32_t)(((t.n + 31) / 32) * ((t.B + 63) / 64));
    case PREP_COLABS: return (uint32_t)((t.n + 63) / 64);
    case PREP_ROWABS: return (uint32_t)((t.n + 3) / 4);
    case PREP_FILL4: return (uint32_t)((t.n + 255) / 256);
    default: return (uint32_t)((t.n * t.B + 255) / 256);
    }
}

void launch_prep(const PrepTask *tasks, int nt, hipStream_t st) {
    PrepArgs a{};
    uint32_t blocks = 0;
    for (int k = 0; k < nt; ++k) {
        const uint32_t nb = prep_blocks(tasks[k]);
        if (nb == 0) continue;
        if (a.nt == PREP_MAX) throw_error(3, "launch_prep: too many tasks (internal error)");
        a.t[a.nt] = tasks[k];
        a.t[a.nt].first = blocks;
        blocks += nb;
        ++a.nt;
    }
    if (blocks == 0) return;
    // named for its task when it holds one (the names of the separate launches)
    static const char *const names[] = {"transpose", "colabs", "rowabs", "fill", "zero_split"};
    ProfScope ps(a.nt == 1 ? names[a.t[0].kind] : "prep", st);
    launch(k_prep, dim3(blocks), dim3(256), 0, st, a);
    SILI_HIP(hipGetLastError());
}

void launch_rowabs(const float *xT, int64_t B, int64_t n, float *acc, hipStream_t st) {
    if (B == 0 || n == 0) return;
    ProfScope ps("rowabs", st);
    launch(k_rowabs, dim3((unsigned)((n + 3) / 4)), dim3(256), 0, st, xT, B, n, acc);
    SILI_HIP(hipGetLastError());
}

void launch_colabs(const float *src, int64_t B, int64_t n, float *acc, hipStream_t st) {
    if (B == 0 || n == 0) return;
    ProfScope ps("colabs", st);
    if (n % 4 == 0 && aligned16(src) && aligned16(acc))
        launch(k_colabs_v4, dim3((unsigned)((n + 63) / 64)), dim3(256), 0, st, src, B, n, acc);
    else
        launch(k_colabs, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, src, B, n, acc);
    SILI_HIP(hipGetLastError());
}

void launch_zero_split_rows(const GatherPlan &p, float *out, int64_t out_ld, int64_t nb, hipStream_t st) {
    if (p.nseg == 0 || nb == 0 || !p.has_split || p.n_split == 0) return;
    ProfScope ps("zero_split", st);
    if (p.n_split * 4 >= p.rows) {
        // most rows split: one streaming fill of the whole output is cheaper
        const int64_t n = nb * out_ld;
        const int64_t n4 = aligned16(out) ? n / 4 : 0;
        if (n4 > 0) launch(k_zero_f4, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, st, reinterpret_cast<float4 *>(out), n4);
        if (n - 4 * n4 > 0) launch(k_zero_f1, dim3((unsigned)((n - 4 * n4 + 255) / 256)), dim3(256), 0, st, out + 4 * n4, n - 4 * n4);
    } else {
        const int64_t n = p.n_split * nb;
        launch(k_zero_split_rows, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, p.split_rows, p.n_split, out,
               out_ld, nb);
    }
    SILI_HIP(hipGetLastError());
}

void launch_densify_full(const int32_t *ptrs, const int32_t *idx, const float *vals, int64_t B, int64_t n,
                         float *dst, float *acc_abs, bool mark_explicit, int64_t nnz, hipStream_t st) {
    if (B == 0 || n == 0) return;
    ProfScope ps("densify", st);
    if (B > DENSIFY_TILE_MAX_B) {
        // a zero fill, then one thread per entry
        const int64_t cnt = B * n;
        const int64_t n4 = aligned16(dst) ? cnt / 4 : 0;
        if (n4 > 0) launch(k_zero_f4, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, st, reinterpret_cast<float4 *>(dst), n4);
        if (cnt - 4 * n4 > 0) launch(k_zero_f1, dim3((unsigned)((cnt - 4 * n4 + 255) / 256)), dim3(256), 0, st, dst + 4 * n4, cnt - 4 * n4);
        if (nnz > 0)
            launch(k_densify_entries, dim3((unsigned)((nnz + 255) / 256)), dim3(256), 0, st, ptrs, idx, vals, B, n, dst,
                   acc_abs, mark_explicit ? 1 : 0);
        SILI_HIP(hipGetLastError());
        return;
    }
    const int64_t R = std::max<int64_t>(1, std::min<int64_t>(256, 2048 / B));
    const size_t lds = (size_t)(R * B) * sizeof(float);
    uint32_t lg = 5;  // lanes per search: 2 * B * 2^lg <= 1024
    while ((2 * B) << lg > 1024) --lg;
    launch(k_densify_tiles, dim3((unsigned)((n + R - 1) / R)), dim3(1024), (uint32_t)lds, st, ptrs, idx, vals, B, n, R,
           lg, dst, acc_abs, mark_explicit ? 1 : 0);
    SILI_HIP(hipGetLastError());
}

void launch_decode(const GatherPlan &p, const ScaleView &sc, int32_t *cols, float *w,
                   uint32_t *rows_out, hipStream_t st) {
    if (p.nseg == 0) return;
    DArgs a{p.seg, p.nseg, p.idx, p.val, sc, cols, w, rows_out};
    launch(k_decode, dim3(blocks_for(p.nseg)), dim3(256), 0, st, a);
    SILI_HIP(hipGetLastError());
}

void launch_decode_b4(const Block4Plan &p, uint32_t *tile_br, uint32_t *tile_bc, hipStream_t st) {
    if (p.nseg == 0) return;
    launch(k_decode_b4, dim3(blocks_for(p.nseg)), dim3(256), 0, st, p.seg, p.nseg, p.idx,
                       tile_br, tile_bc);
    SILI_HIP(hipGetLastError());
}

}  // namespace sili
