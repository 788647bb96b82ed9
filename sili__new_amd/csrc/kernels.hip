// kernels.hip -- gfx950 kernels of the FP4 delta-CSR layer's hot path.
//
//   k_gather     scattered store, out[b,row] = sum_e w_e * in[col_e, b]
//                (forward on the shadow store, grad-input on the canonical one)
//   k_gather_b4  block4 contribution of the same, 4 output rows per block row
//   k_sddmm      nnz-sampled grad-W over the scattered store
//   k_sddmm_b4   nnz-sampled grad-W over every block4 slot
//   k_transpose  [B,n] -> [n,B] activations, fused sum_b |x| accumulators
//   k_densify    CSR activations -> dense feature-major
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
};

template <int G, int KB, int SKIP>
__global__ __launch_bounds__(256) void k_gather(GArgs a) {
    __shared__ uint32_t s_col[WAVES][64];
    __shared__ float s_w[WAVES][64];
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const int64_t si = (int64_t)blockIdx.x * WAVES + wave;
    if (si >= a.nseg) return;
    const SegDesc sd = a.seg[si];
    constexpr uint32_t BL = 64u / G;
    const uint32_t g = lane / BL, bl = lane % BL;
    const uint32_t row = sd.row;
    float acc[KB];
#pragma unroll
    for (int k = 0; k < KB; ++k) acc[k] = 0.0f;
    uint32_t pos = sd.byte_begin, carry = sd.base_col, ebase = sd.elem_begin;
    const uint32_t end = sd.byte_end;
    while (pos < end) {
        const Chunk ch = decode_chunk(a.idx, pos, end, carry);
        if (ch.T == 0ull) break;  // malformed stream: never spin
        if (ch.term) {
            const uint32_t code = (uint32_t)a.val[ebase + ch.rank] >> 4;
            s_col[wave][ch.rank] = ch.col;
            s_w[wave][ch.rank] = fp4_decode(code) * scale_at(a.sc, row, ch.col);
        }
        wave_lds_sync();
        const uint32_t n = (uint32_t)__popcll(ch.T);
        for (uint32_t j = 0; j < n; j += G) {
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
                if (sd.split) atomicAdd(o, acc[k]);
                else *o = acc[k];
            }
        }
    }
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
                    if (sd.split) atomicAdd(o, acc[li][k]);
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
};

// gw[e] = sum_b xT[row,b] * gT[col_e,b]; each terminator lane owns one entry
// and streams its gT row (float4 along b), xT[row,:] is staged in LDS.
__global__ __launch_bounds__(256) void k_sddmm(SArgs a) {
    extern __shared__ __align__(16) float s_x[];  // [WAVES][B]
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const int64_t si = (int64_t)blockIdx.x * WAVES + wave;
    if (si >= a.nseg) return;
    const SegDesc sd = a.seg[si];
    const int64_t B = a.B;
    float *sx = s_x + (int64_t)wave * B;
    for (int64_t b = lane; b < B; b += 64) sx[b] = a.xT[(int64_t)sd.row * B + b];
    wave_lds_sync();
    uint32_t pos = sd.byte_begin, carry = sd.base_col, ebase = sd.elem_begin;
    const uint32_t end = sd.byte_end;
    const bool vec4 = (B & 3) == 0;
    while (pos < end) {
        const Chunk ch = decode_chunk(a.idx, pos, end, carry);
        if (ch.T == 0ull) break;
        if (ch.term) {
            const float *gr = a.gT + (int64_t)ch.col * B;
            float acc = 0.0f;
            if (vec4) {
                float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
                for (int64_t b = 0; b < B; b += 4) {
                    const float4 gv = *reinterpret_cast<const float4 *>(gr + b);
                    const float4 xv = *reinterpret_cast<const float4 *>(sx + b);
                    a0 = __builtin_fmaf(xv.x, gv.x, a0);
                    a1 = __builtin_fmaf(xv.y, gv.y, a1);
                    a2 = __builtin_fmaf(xv.z, gv.z, a2);
                    a3 = __builtin_fmaf(xv.w, gv.w, a3);
                }
                acc = (a0 + a1) + (a2 + a3);
            } else {
                for (int64_t b = 0; b < B; ++b) acc = __builtin_fmaf(sx[b], gr[b], acc);
            }
            a.gw[ebase + ch.rank] = acc;
        }
        carry = chunk_advance(ch, pos, ebase);
    }
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
                    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
                    for (int64_t b = 0; b < B; b += 4) {
                        const float4 gv = *reinterpret_cast<const float4 *>(gr + b);
                        const float4 xv = *reinterpret_cast<const float4 *>(xr + b);
                        a0 = __builtin_fmaf(xv.x, gv.x, a0);
                        a1 = __builtin_fmaf(xv.y, gv.y, a1);
                        a2 = __builtin_fmaf(xv.z, gv.z, a2);
                        a3 = __builtin_fmaf(xv.w, gv.w, a3);
                    }
                    acc = (a0 + a1) + (a2 + a3);
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

// [B, n] -> [n, B] through a 64x65 LDS tile; optional acc[j] += sum_b |x[b,j]|.
__global__ __launch_bounds__(256) void k_transpose(const float *__restrict__ src, int64_t B,
                                                   int64_t n, float *__restrict__ dst,
                                                   float *__restrict__ acc) {
    __shared__ float tile[64][65];
    const int64_t j0 = (int64_t)blockIdx.x * 64, b0 = (int64_t)blockIdx.y * 64;
    const uint32_t tx = threadIdx.x & 63u, ty = threadIdx.x >> 6;  // 64 x 4
    float part = 0.0f;
    for (uint32_t i = ty; i < 64u; i += 4u) {
        const int64_t b = b0 + i, j = j0 + tx;
        float v = 0.0f;
        if (b < B && j < n) v = src[b * n + j];
        tile[i][tx] = v;
        part += __builtin_fabsf(v);
    }
    if (acc) {
        __shared__ float red[4][64];
        red[ty][tx] = part;
        __syncthreads();
        if (ty == 0 && j0 + tx < n) {
            const float s = (red[0][tx] + red[1][tx]) + (red[2][tx] + red[3][tx]);
            atomicAdd(acc + j0 + tx, s);
        }
    }
    __syncthreads();
    for (uint32_t i = ty; i < 64u; i += 4u) {
        const int64_t j = j0 + i, b = b0 + tx;
        if (j < n && b < B) dst[j * B + b] = tile[tx][i];
    }
}

__global__ __launch_bounds__(256) void k_colabs(const float *__restrict__ src, int64_t B, int64_t n,
                                                float *__restrict__ acc) {
    const int64_t j = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (j >= n) return;
    float s = 0.0f;
    for (int64_t b = 0; b < B; ++b) s += __builtin_fabsf(src[b * n + j]);
    acc[j] += s;
}

__global__ __launch_bounds__(256) void k_densify(const int32_t *__restrict__ ptrs,
                                                 const int32_t *__restrict__ idx,
                                                 const float *__restrict__ vals, int64_t B,
                                                 int64_t n, float *__restrict__ dst,
                                                 float *__restrict__ acc_abs, int mark) {
    const int64_t b = blockIdx.x;
    const int64_t p0 = ptrs[b], p1 = ptrs[b + 1];
    for (int64_t p = p0 + threadIdx.x; p < p1; p += 256) {
        const int64_t j = idx[p];
        if (j < 0 || j >= n) continue;  // host validated; never write out of bounds
        float v = vals[p];
        if (acc_abs) atomicAdd(acc_abs + j, __builtin_fabsf(v));
        if (mark && __builtin_bit_cast(uint32_t, v) == 0u) v = -0.0f;
        dst[j * B + b] = v;
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
    const int64_t si = (int64_t)blockIdx.x * WAVES + wave;
    if (si >= a.nseg) return;
    const SegDesc sd = a.seg[si];
    uint32_t pos = sd.byte_begin, carry = sd.base_col, ebase = sd.elem_begin;
    const uint32_t end = sd.byte_end;
    while (pos < end) {
        const Chunk ch = decode_chunk(a.idx, pos, end, carry);
        if (ch.T == 0ull) break;
        if (ch.term) {
            const uint32_t e = ebase + ch.rank;
            if (a.cols) a.cols[e] = (int32_t)ch.col;
            if (a.w) a.w[e] = fp4_decode((uint32_t)a.val[e] >> 4) * scale_at(a.sc, sd.row, ch.col);
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
        case SKIP_ZERO: hipLaunchKernelGGL((k_gather<G, KB, SKIP_ZERO>), grid, block, 0, st, a); break;
        case SKIP_POSZERO: hipLaunchKernelGGL((k_gather<G, KB, SKIP_POSZERO>), grid, block, 0, st, a); break;
        default: hipLaunchKernelGGL((k_gather<G, KB, SKIP_NONE>), grid, block, 0, st, a); break;
    }
}

template <int G, int KB>
void gather_b4_dispatch_skip(const BArgs &a, int skip, hipStream_t st) {
    const dim3 grid(blocks_for(a.nseg)), block(256);
    switch (skip) {
        case SKIP_ZERO: hipLaunchKernelGGL((k_gather_b4<G, KB, SKIP_ZERO>), grid, block, 0, st, a); break;
        case SKIP_POSZERO: hipLaunchKernelGGL((k_gather_b4<G, KB, SKIP_POSZERO>), grid, block, 0, st, a); break;
        default: hipLaunchKernelGGL((k_gather_b4<G, KB, SKIP_NONE>), grid, block, 0, st, a); break;
    }
}

}  // namespace

void launch_gather(const GatherPlan &p, const ScaleView &sc, const float *in, int64_t in_ld,
                   float *out, int64_t out_ld, int64_t nb_total, int skip, hipStream_t st) {
    if (p.nseg == 0 || nb_total == 0) return;
    for (int64_t b0 = 0; b0 < nb_total; b0 += 512) {
        const int64_t nb = nb_total - b0 < 512 ? nb_total - b0 : 512;
        GArgs a{p.seg, p.nseg, p.idx, p.val, sc, in + b0, in_ld, out + b0 * out_ld, out_ld, nb};
        if (nb == 1) gather_dispatch_skip<64, 1>(a, skip, st);
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
                  hipStream_t st) {
    if (p.nseg == 0) return;
    SArgs a{p.seg, p.nseg, p.idx, xT, gT, B, gw};
    const size_t lds = sizeof(float) * (size_t)WAVES * (size_t)B;
    if (lds > 64 * 1024) throw_error(1, "sampled grad-W: batch too large for one launch (max 4096)");
    hipLaunchKernelGGL(k_sddmm, dim3(blocks_for(p.nseg)), dim3(256), lds, st, a);
    SILI_HIP(hipGetLastError());
}

void launch_sddmm_b4(const Block4Plan &p, const uint32_t *, const float *xT, const float *gT,
                     int64_t B, float *gw, hipStream_t st) {
    if (p.nseg == 0) return;
    SBArgs a{p.seg, p.nseg, p.idx, p.rows, p.cols, xT, gT, B, gw};
    const size_t lds = sizeof(float) * (size_t)WAVES * 4u * (size_t)B;
    if (lds > 64 * 1024) throw_error(1, "block4 sampled grad-W: batch too large (max 1024)");
    hipLaunchKernelGGL(k_sddmm_b4, dim3(blocks_for(p.nseg)), dim3(256), lds, st, a);
    SILI_HIP(hipGetLastError());
}

void launch_transpose(const float *src, int64_t B, int64_t n, float *dst, float *acc,
                      hipStream_t st) {
    if (B == 0 || n == 0) return;
    const dim3 grid((unsigned)((n + 63) / 64), (unsigned)((B + 63) / 64));
    hipLaunchKernelGGL(k_transpose, grid, dim3(256), 0, st, src, B, n, dst, acc);
    SILI_HIP(hipGetLastError());
}

void launch_colabs(const float *src, int64_t B, int64_t n, float *acc, hipStream_t st) {
    if (B == 0 || n == 0) return;
    hipLaunchKernelGGL(k_colabs, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, src, B, n, acc);
    SILI_HIP(hipGetLastError());
}

void launch_densify(const int32_t *ptrs, const int32_t *idx, const float *vals, int64_t B,
                    int64_t n, float *dst, float *acc_abs, bool mark_explicit, hipStream_t st) {
    if (B == 0) return;
    hipLaunchKernelGGL(k_densify, dim3((unsigned)B), dim3(256), 0, st, ptrs, idx, vals, B, n, dst,
                       acc_abs, mark_explicit ? 1 : 0);
    SILI_HIP(hipGetLastError());
}

void launch_decode(const GatherPlan &p, const ScaleView &sc, int32_t *cols, float *w,
                   uint32_t *rows_out, hipStream_t st) {
    if (p.nseg == 0) return;
    DArgs a{p.seg, p.nseg, p.idx, p.val, sc, cols, w, rows_out};
    hipLaunchKernelGGL(k_decode, dim3(blocks_for(p.nseg)), dim3(256), 0, st, a);
    SILI_HIP(hipGetLastError());
}

void launch_decode_b4(const Block4Plan &p, uint32_t *tile_br, uint32_t *tile_bc, hipStream_t st) {
    if (p.nseg == 0) return;
    hipLaunchKernelGGL(k_decode_b4, dim3(blocks_for(p.nseg)), dim3(256), 0, st, p.seg, p.nseg, p.idx,
                       tile_br, tile_bc);
    SILI_HIP(hipGetLastError());
}

}  // namespace sili
