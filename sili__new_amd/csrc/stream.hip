// stream.hip -- batch-1 gather over a padded stream copy ("stream" kernels).
//
// out[row] = sum over the row's entries of dec(code) * S(row, col) * in[col]
// for one input vector: the forward y = W x over the shadow store, or
// dx = W^T g over the canonical one (linear_disldo.hpp:68-345 / :962-1951 at
// batch 1).  The per-row segment kernels give every row its own work items,
// so a row slightly longer than a work item costs two wave passes.  Here the
// work is cut into fixed 1024-byte windows of a padded copy of the store's
// index stream (DStream), so every wave pass decodes 64 x 16 index bytes
// whatever the row lengths:
//   - rows start on 16-byte boundaries (zero-delta padding entries in front,
//     columns shifted by one so that shifted column 0 is a zero input slot):
//     each lane's 16 bytes belong to one row, and the per-entry work is one
//     add, one LDS (or cache) read, one FP4 conversion and one FMA,
//   - value bytes run in parallel with index bytes (val[p] belongs to the
//     entry whose varint ends at byte p), so no entry count is needed to
//     find them,
//   - the running column of each lane comes from a segmented wave scan of
//     the lanes' delta sums (byte sums by v_sad_u8), restarted at row
//     starts; per-row partial sums are combined by a second segmented scan
//     and leave as one atomic add per row piece (the output is zeroed first).
// A window whose bytes are all one-byte varints takes a decode without
// continuation handling; any other window (long deltas, the stream's partial
// last window) takes the general decode.
//
// XLDS: the block first stages in[c] * ent_scale[c] in LDS (slot c + 1,
// slot 0 = 0); otherwise in and the column scale come through buffer loads
// whose out-of-range reads return 0.  The FP4 code is expanded by
// v_cvt_scalef32_pk_f32_fp4 (OCP E2M1: the reference decode for every code
// but 8, which never reaches these kernels: they serve only layers without
// non-finite weights, SKIP_NONE).
#include "layer.hpp"
#include "wave.hpp"

#include <algorithm>
#include <map>
#include <mutex>
#include <tuple>

namespace sili {

namespace {

constexpr unsigned TPB = 256;
constexpr uint32_t BPL = 16;  // index bytes per lane

inline unsigned nblk(int64_t n) { return (unsigned)((n + TPB - 1) / TPB); }

// ---- building the stream copy ----------------------------------------------

// Where column block k of row r begins and ends in the row's index bytes:
// first entry's byte offset s, varint length lf, column c and entry index ei
// (in the store), and the byte offset e where the block's entries end.
// e == 0: the row has no entry in the block.
struct BlkMeta {
    uint32_t s, lf, e, c, ei;
};

// Pass 1: one wave per row.
__global__ __launch_bounds__(256) void k_spb_meta(const uint32_t *__restrict__ bs, const uint32_t *__restrict__ es,
                                                  const uint8_t *__restrict__ idx, int64_t rows, uint32_t cb,
                                                  BlkMeta *__restrict__ meta) {
    const int64_t r = (int64_t)blockIdx.x * 4 + uniform(threadIdx.x >> 6);
    if (r >= rows) return;
    const uint32_t lane = lane_id();
    const uint32_t b = bs[r], n = bs[r + 1] - b;
    if (n == 0) return;
    const uint8_t *row = idx + b;
    uint32_t off = 0, carry = 0, ebase = es[r];
    uint32_t kopen = 0xFFFFFFFFu;  // block of the entry before the chunk
    while (off < n) {
        const Chunk ch = decode_chunk(row, off, n, carry);
        if (ch.T == 0ull) break;
        const uint64_t below = ch.T & ((1ull << lane) - 1ull);
        const int pl = below ? 63 - (int)__clzll(below) : -1;  // previous entry's last byte in the chunk
        const uint32_t kb = ch.col / cb;
        const uint32_t kpl = (uint32_t)__shfl((int)kb, pl < 0 ? 0 : pl, 64);
        const uint32_t kp = pl < 0 ? kopen : kpl;
        uint64_t F = __ballot(ch.term && kb != kp);  // entries that open a block
        while (F) {
            const int fl = __builtin_ctzll(F);
            F &= F - 1ull;
            const uint32_t kf = (uint32_t)__builtin_amdgcn_readlane((int)kb, fl);
            const uint32_t cf = (uint32_t)__builtin_amdgcn_readlane((int)ch.col, fl);
            const int pf = __builtin_amdgcn_readlane(pl, fl);
            const uint32_t rk = (uint32_t)__builtin_amdgcn_readlane((int)ch.rank, fl);
            const uint32_t s0 = off + (uint32_t)(pf + 1);
            if (lane == 0u) {
                BlkMeta &m = meta[(int64_t)kf * rows + r];
                m.s = s0;
                m.lf = (uint32_t)(fl - pf);
                m.c = cf;
                m.ei = ebase + rk;
                if (kopen != 0xFFFFFFFFu) meta[(int64_t)kopen * rows + r].e = s0;
            }
            kopen = kf;
        }
        carry = chunk_advance(ch, off, ebase);
    }
    if (lane == 0u && kopen != 0xFFFFFFFFu) meta[(int64_t)kopen * rows + r].e = n;
}

// Padded length of block k of row r (first delta re-encoded for the shifted
// column, rounded up to 16); lens / nonempty are [K][rows + 1].
__global__ void k_spb_len(const BlkMeta *__restrict__ meta, int64_t rows, int K, uint32_t cb,
                          uint32_t *__restrict__ len, uint32_t *__restrict__ nonempty) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i >= (int64_t)K * (rows + 1)) return;
    const int64_t k = i / (rows + 1), r = i - k * (rows + 1);
    uint32_t L = 0;
    if (r < rows) {
        const BlkMeta m = meta[k * rows + r];
        if (m.e) L = (uleb_len(m.c - (uint32_t)k * cb + 1u) + (m.e - m.s - m.lf) + 15u) & ~15u;
    }
    len[i] = L;
    nonempty[i] = L ? 1u : 0u;
}

__global__ void k_sp_ne(const uint32_t *__restrict__ nonempty, const uint32_t *__restrict__ pos,
                        const uint32_t *__restrict__ pstart, int64_t rows, uint32_t *__restrict__ ne_row,
                        uint32_t *__restrict__ ne_start) {
    const int64_t r = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (r > rows) return;
    if (r == rows) {
        ne_start[pos[r]] = pstart[r];  // sentinel: the block's bytes
        return;
    }
    if (nonempty[r]) {
        ne_row[pos[r]] = (uint32_t)r;
        ne_start[pos[r]] = pstart[r];
    }
}

// Pass 2: one wave per (block, row): copy the block's entries of the row into
// the block's padded stream (first delta re-encoded for the shifted column,
// value bytes placed at their terminators) and write the carry of every
// window of the block that starts inside the row's padded range.
__global__ __launch_bounds__(256) void k_spb_copy(const uint32_t *__restrict__ bs, const uint8_t *__restrict__ idx,
                                                  const uint8_t *__restrict__ val, const BlkMeta *__restrict__ meta,
                                                  const uint32_t *__restrict__ pstart, int64_t rows, uint32_t c0,
                                                  uint8_t *__restrict__ sidx, uint8_t *__restrict__ sval,
                                                  WinDesc *__restrict__ win) {
    const int64_t r = (int64_t)blockIdx.x * 4 + uniform(threadIdx.x >> 6);
    if (r >= rows) return;
    const uint32_t lane = lane_id();
    const BlkMeta m = meta[r];
    if (m.e == 0u) return;
    const uint32_t P = pstart[r], Lr = pstart[r + 1] - P;
    const uint32_t v1 = m.c - c0 + 1u, l1 = uleb_len(v1);
    const uint32_t body = m.e - m.s - m.lf;  // bytes after the first entry
    const uint32_t z = Lr - (l1 + body);      // padding entries in front
    const uint32_t D = P + z + l1;            // padded position of row byte s + lf
    if (lane < l1) sidx[P + z + lane] = (uint8_t)(((v1 >> (7u * lane)) & 0x7Fu) | (lane + 1u < l1 ? 0x80u : 0u));
    if (lane == 0u) sval[D - 1u] = val[m.ei];
    // a window starting before the first entry's last byte: only padding
    // entries (shifted column 0) precede it
    const uint32_t w_pad = (P + WIN_BYTES - 1u) / WIN_BYTES * WIN_BYTES;
    if (lane == 0u && w_pad < D) win[w_pad / WIN_BYTES].carry = 0u;
    const uint8_t *row = idx + bs[r];
    const uint32_t o0 = m.s + m.lf;
    uint32_t off = o0, carry = m.c, ebase = m.ei + 1u;
    while (off < m.e) {
        const Chunk ch = decode_chunk(row, off, m.e, carry);
        if (ch.T == 0ull) break;
        const uint32_t hi = 63u - (uint32_t)__clzll(ch.T);  // last byte of the chunk's last entry
        const uint32_t d0 = D + off - o0;                   // padded position of byte `off`
        if (lane <= hi) {
            sidx[d0 + lane] = row[off + lane];
            if (ch.term) sval[d0 + lane] = val[ebase + ch.rank];
        }
        // a window starting inside the chunk's bytes [d0, d0 + hi]
        const uint32_t ws = (d0 + WIN_BYTES - 1u) / WIN_BYTES * WIN_BYTES;
        if (ws <= d0 + hi) {
            const uint64_t before = ch.T & ((1ull << (ws - d0)) - 1ull);
            uint32_t c = carry - c0 + 1u;
            if (before) c = (uint32_t)__shfl((int)ch.col, 63 - (int)__clzll(before), 64) - c0 + 1u;
            if (lane == 0u) win[ws / WIN_BYTES].carry = c;
        }
        carry = chunk_advance(ch, off, ebase);
    }
}

// rs_lo and the row-start mask of every window of a block: the first
// non-empty row starting at or after the window, and the lanes on which the
// rows starting inside it begin.
__global__ void k_sp_rs(const uint32_t *__restrict__ ne_start, int64_t n_ne, int64_t nwin,
                        WinDesc *__restrict__ win) {
    const int64_t w = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (w > nwin) return;
    if (w == nwin) {
        win[w] = WinDesc{0u, (uint32_t)n_ne, 0u, 0u};
        return;
    }
    const uint64_t b0 = (uint64_t)w * WIN_BYTES;
    int64_t lo = 0, hi = n_ne;
    while (lo < hi) {
        const int64_t mid = (lo + hi) >> 1;
        if ((uint64_t)ne_start[mid] < b0) lo = mid + 1;
        else hi = mid;
    }
    uint64_t mask = 0;
    for (int64_t k = lo; k < n_ne && (uint64_t)ne_start[k] < b0 + WIN_BYTES; ++k)
        mask |= 1ull << (((uint64_t)ne_start[k] - b0) / BPL);
    win[w].rs_lo = (uint32_t)lo;
    win[w].mask_lo = (uint32_t)mask;
    win[w].mask_hi = (uint32_t)(mask >> 32);
}

// ---- the gather ------------------------------------------------------------

struct StreamArgs {
    const WinDesc *win;          // nwin + 1
    int64_t nwin;
    const uint8_t *idx, *val;    // padded stream
    const uint32_t *ne_row;      // non-empty rows, ascending
    uint32_t nbytes;
    uint32_t n_ne;               // non-empty rows
    const float *in;             // in[c * in_ld + j], c < nx, j < NB (this pass)
    uint32_t in_ld;
    const float *ent;            // column scale (NULL: ones)
    const float *rsc;            // row scale (NULL: ones)
    uint32_t nx;
    uint32_t rows;               // rows of the store
    float *out;                  // out[j * out_ld + row], zeroed beforehand
    int64_t out_ld;
};

// Buffer resources of one launch.  Every memory access of the window loop is
// a buffer access whose out-of-range offsets read 0 (atomics: are dropped),
// so each pass of the loop issues the same loads on every path and the
// compiler's wait counts stay exact: a window's loads are waited for one
// window after they were issued, never together with the next window's.
struct StreamRsrc {
    __amdgpu_buffer_rsrc_t idx, val, ner, win, rsc, out, in, ent;
};

__device__ __forceinline__ uint4 buffer_load_u4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
}
// The same, non-temporal (cache policy nt): for the stream's bytes, which a
// pass reads once.
__device__ __forceinline__ uint4 buffer_load_u4_nt(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 2));
}
__device__ __forceinline__ uint32_t buffer_load_u1(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0);
}

// A window's descriptor (WinDesc), uniform.
struct WinMeta {
    uint32_t carry, rs_lo, mask_lo, mask_hi;
};
// The same as loaded (per lane, before readfirstlane).
struct WinRaw {
    uint4 d;
};
// One window's per-lane loads: the lane's 16 index and 16 value bytes, the
// index dword before the window (0 for the first), and Rr = entry
// rs_lo - h + lane of the list of non-empty rows for lanes below
// popcount(mask) + h, where h = 1 when no row starts at the window's first
// byte (then lane 0 holds the row that byte belongs to), else 0.
struct WinData {
    uint32_t i[4], v[4], ip;
    uint32_t Rr;
};

__device__ __forceinline__ void issue_meta(const StreamRsrc &r, int64_t w, WinRaw &q) {
    q.d = buffer_load_u4(r.win, (uint32_t)w * 16u);
}
__device__ __forceinline__ WinMeta uniform_meta(const WinRaw &q) {
    return WinMeta{uniform(q.d.x), uniform(q.d.y), uniform(q.d.z), uniform(q.d.w)};
}
__device__ __forceinline__ uint32_t head_missing(const WinMeta &m) { return (m.mask_lo & 1u) ^ 1u; }
// Windows at or past nwin read zeros (no rows, no bytes).
__device__ __forceinline__ void issue_data(const StreamRsrc &r, int64_t w, const WinMeta &m, WinData &d) {
    const uint32_t lane = lane_id();
    const uint32_t b0 = (uint32_t)w * WIN_BYTES;
    const uint4 iw = buffer_load_u4_nt(r.idx, b0 + BPL * lane);
    const uint4 vw = buffer_load_u4_nt(r.val, b0 + BPL * lane);
    d.i[0] = iw.x;
    d.i[1] = iw.y;
    d.i[2] = iw.z;
    d.i[3] = iw.w;
    d.v[0] = vw.x;
    d.v[1] = vw.y;
    d.v[2] = vw.z;
    d.v[3] = vw.w;
    d.ip = buffer_load_u1(r.idx, b0 ? b0 - 4u : OOB_OFFSET);
    // rows starting here (<= 64; h = 1 only when lane 0 starts none, so
    // nr + h <= 64)
    const uint32_t h = head_missing(m);
    const uint32_t nr = (uint32_t)__builtin_popcount(m.mask_lo) + (uint32_t)__builtin_popcount(m.mask_hi);
    d.Rr = buffer_load_u1(r.ner, lane < nr + h ? (m.rs_lo - h + lane) * 4u : OOB_OFFSET);
}

// Weight code of value byte K (0..3) of dw: the high nibble.  The conversion
// yields both nibbles of the byte, low nibble first.
template <int K>
__device__ __forceinline__ float fp4_code_hi(uint32_t dw) {
    return __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(dw, 1.0f, K)[1];
}
__device__ __forceinline__ float fp4_code_hi_byte(uint32_t dw, int k) {
    switch (k & 3) {
        case 0: return fp4_code_hi<0>(dw);
        case 1: return fp4_code_hi<1>(dw);
        case 2: return fp4_code_hi<2>(dw);
        default: return fp4_code_hi<3>(dw);
    }
}

template <int NB>
struct XVec {
    float v[NB];
};

// The NB inputs at shifted column c (0: the zero slot).  XLDS: slot c holds
// NB floats; otherwise buffer loads of in[(c - 1) * in_ld + j] times the
// column scale (c = 0 wraps out of range and reads 0; the scale load is made
// even without scales, against a zero-sized range).
template <int NB, bool XLDS>
__device__ __forceinline__ XVec<NB> stream_x(const StreamArgs &a, const StreamRsrc &r, const float *s_x,
                                             uint32_t c) {
    XVec<NB> x;
    if constexpr (XLDS) {
        const float *p = s_x + c * NB;
        if constexpr (NB == 1) {
            x.v[0] = p[0];
        } else if constexpr (NB == 2) {
            const float2 t = *reinterpret_cast<const float2 *>(p);
            x.v[0] = t.x;
            x.v[1] = t.y;
        } else {
#pragma unroll
            for (int q = 0; q < NB / 4; ++q) {
                const float4 t = reinterpret_cast<const float4 *>(p)[q];
                x.v[4 * q] = t.x;
                x.v[4 * q + 1] = t.y;
                x.v[4 * q + 2] = t.z;
                x.v[4 * q + 3] = t.w;
            }
        }
    } else {
        const uint32_t off = (c - 1u) * a.in_ld * 4u;
        if constexpr (NB >= 4) {
#pragma unroll
            for (int q = 0; q < NB / 4; ++q) {
                const float4 t = buffer_load_f4(r.in, off + 16u * (uint32_t)q);
                x.v[4 * q] = t.x;
                x.v[4 * q + 1] = t.y;
                x.v[4 * q + 2] = t.z;
                x.v[4 * q + 3] = t.w;
            }
        } else {
#pragma unroll
            for (int j = 0; j < NB; ++j) x.v[j] = buffer_load_f1(r.in, off + 4u * (uint32_t)j);
        }
        const float e = buffer_load_f1(r.ent, (c - 1u) * 4u);
        if (a.ent) {
#pragma unroll
            for (int j = 0; j < NB; ++j) x.v[j] *= e;
        }
    }
    return x;
}

// Segmented inclusive scan of NB values (the wave_seg_scan ladder) whose
// segments begin at the lanes of the uniform mask S.  The flag each step
// selects on depends on S alone, so the ladder is built with scalar
// operations: F |= F moved the way the step moves values (row_shr n: up by
// n inside each 16-lane row; row_bcast15: lane 15 / 47 into rows 1 / 3;
// row_bcast31: lane 31 into rows 2 and 3), and each step's select reads the
// lane's bit of F directly as its condition.
template <int NB, int CTRL, int RM>
__device__ __forceinline__ void seg_step_mask(float (&v)[NB], uint64_t F) {
    const bool f = __builtin_amdgcn_inverse_ballot_w64(F);
#pragma unroll
    for (int j = 0; j < NB; ++j) {
        const float t = dpp_f32<CTRL, RM>(v[j]);
        v[j] = f ? v[j] : v[j] + t;
    }
}
template <int NB>
__device__ __forceinline__ void wave_seg_scan_mask(float (&v)[NB], uint64_t S) {
    uint64_t F = S;
    seg_step_mask<NB, DPP_ROW_SHR1, 0xF>(v, F);
    F |= (F << 1) & 0xFFFEFFFEFFFEFFFEull;
    seg_step_mask<NB, DPP_ROW_SHR2, 0xF>(v, F);
    F |= (F << 2) & 0xFFFCFFFCFFFCFFFCull;
    seg_step_mask<NB, DPP_ROW_SHR4, 0xF>(v, F);
    F |= (F << 4) & 0xFFF0FFF0FFF0FFF0ull;
    seg_step_mask<NB, DPP_ROW_SHR8, 0xF>(v, F);
    F |= (F << 8) & 0xFF00FF00FF00FF00ull;
    seg_step_mask<NB, DPP_ROW_BCAST15, 0xA>(v, F);
    F |= (((F >> 15) & 1ull) ? 0x00000000FFFF0000ull : 0ull) | (((F >> 47) & 1ull) ? 0xFFFF000000000000ull : 0ull);
    seg_step_mask<NB, DPP_ROW_BCAST31, 0xC>(v, F);
}

// Decode and multiply-adds of window w (descriptor m, loads d) for the
// lane: acc[j] = sum over the entries in its 16 bytes of weight * input j.
// Inputs through the cache at one or two columns (EARLY) are loaded here
// before the data loads of window wn, which this then issues; otherwise the
// caller issued them.  FAST: every byte is a one-byte varint and none
// continues from the window before.
template <int NB, bool XLDS, bool FAST>
__device__ __forceinline__ void window_body(const StreamArgs &a, const StreamRsrc &r, const float *s_x,
                                            const WinMeta &m, const WinData &d, uint32_t b0, bool hs,
                                            int64_t wn, const WinMeta &mN, WinData &dN, float (&acc)[NB]) {
    const uint32_t lane = lane_id();
    // deltas of the entries ending at each byte (0 where no entry ends)
    uint32_t full = 0;
    uint32_t dv[BPL];
    uint32_t tmask = 0xFFFFu;
    if constexpr (FAST) {
#pragma unroll
        for (int k = 0; k < 4; ++k) full = __builtin_amdgcn_sad_u8(d.i[k], 0u, full);
    } else {
        const uint32_t nb = min(a.nbytes - b0, WIN_BYTES);
        // the previous 4 bytes: the previous lane's, or those before the window
        const uint32_t pw0 = (uint32_t)__shfl_up((int)d.i[3], 1, 64);
        const uint32_t pw = lane ? pw0 : d.ip;
        uint32_t k = 0;  // trailing continuation bytes before this lane (a varint ending here)
#pragma unroll
        for (int i = 3; i >= 0; --i) {
            const bool cont = ((pw >> (8 * i + 7)) & 1u) != 0u;
            k = (k == 3u - (uint32_t)i && cont) ? k + 1u : k;
        }
        uint32_t va = 0, shift = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const bool use = (uint32_t)i >= 4u - k;
            va = use ? (va | (((pw >> (8 * i)) & 0x7Fu) << shift)) : va;
            shift = use ? shift + 7u : shift;
        }
        tmask = 0;
#pragma unroll
        for (int i = 0; i < (int)BPL; ++i) {
            const uint32_t b = (d.i[i >> 2] >> (8 * (i & 3))) & 0xFFu;
            const bool valid = BPL * lane + (uint32_t)i < nb;
            va |= (b & 0x7Fu) << (shift < 32u ? shift : 0u);
            const bool term = valid && (b & 0x80u) == 0u;
            dv[i] = term ? va : 0u;
            tmask |= term ? (1u << i) : 0u;
            full += dv[i];
            va = term ? 0u : va;
            shift = term ? 0u : shift + 7u;
        }
    }

    // shifted column entering the lane: E = carry (unless a row starts at
    // lane 0) plus the delta sums of the lanes before, minus E at the
    // latest row start at or before the lane (E never decreases, so a
    // running maximum over the row-start lanes finds it)
    const uint32_t seed = full + ((lane == 0u && !hs) ? m.carry : 0u);
    const uint32_t E = wave_incl_scan(seed) - full;
    const uint32_t col0 = E - wave_max_scan(hs ? E : 0u);

    // inputs through the cache (one or two columns): loaded before the next
    // window's data, so waiting for them does not wait for that
    constexpr bool EARLY = !XLDS && NB <= 2;
    XVec<NB> xe[EARLY ? BPL : 1];
    if constexpr (EARLY) {
        uint32_t c = col0;
#pragma unroll
        for (int i = 0; i < (int)BPL; ++i) {
            if constexpr (FAST) c += (d.i[i >> 2] >> (8 * (i & 3))) & 0xFFu;
            else c += dv[i];
            const bool t = FAST || ((tmask >> i) & 1u);
            xe[i] = stream_x<NB, false>(a, r, s_x, t ? c : 0u);
        }
        issue_data(r, wn, mN, dN);
        __builtin_amdgcn_sched_barrier(0);
    }

#pragma unroll
    for (int j = 0; j < NB; ++j) acc[j] = 0.0f;
    uint32_t c = col0;
#pragma unroll
    for (int i = 0; i < (int)BPL; ++i) {
        if constexpr (FAST) c += (d.i[i >> 2] >> (8 * (i & 3))) & 0xFFu;
        else c += dv[i];
        const bool t = FAST || ((tmask >> i) & 1u);
        // a byte ending no entry has value byte 0 (weight 0) and reads the
        // zero slot
        const float wq = fp4_code_hi_byte(d.v[i >> 2], i);
        XVec<NB> x;
        if constexpr (EARLY) x = xe[i];
        else x = stream_x<NB, XLDS>(a, r, s_x, t ? c : 0u);
#pragma unroll
        for (int j = 0; j < NB; ++j) acc[j] = __builtin_fmaf(wq, x.v[j], acc[j]);
    }
}

// Window w (descriptor m, loads d): out[j*out_ld + row] += its row pieces.
// Its memory operations, in this order: the descriptor load of window wn2
// (into qn, after qn's descriptor of window wn is read into mN), the row
// scales, the data loads of window wn (into dN), the output atomics.  With
// the counter of memory operations completing in order, reading a
// descriptor or a row scale then never waits for data loads issued after
// it; and the loads sit in straight-line code (the decode branch holds
// none, or the same ones on both sides), which keeps the compiler's wait
// counts exact.
template <int NB, bool XLDS>
__device__ __forceinline__ void run_window(const StreamArgs &a, const StreamRsrc &r, int64_t w, const WinMeta &m,
                                           const WinData &d, int64_t wn, int64_t wn2, WinRaw &qn, WinMeta &mN,
                                           WinData &dN, const float *s_x) {
    const uint32_t b0 = (uint32_t)w * WIN_BYTES;
    mN = uniform_meta(qn);
    issue_meta(r, wn2, qn);
    __builtin_amdgcn_sched_barrier(0);

    // the lane's row: rows starting at or before the lane (inclusive count
    // from the row-start mask) pick its entry of the row list
    const uint64_t S = ((uint64_t)m.mask_hi << 32) | m.mask_lo;
    const bool hs = __builtin_amdgcn_inverse_ballot_w64(S);
    const uint32_t cnt = __builtin_amdgcn_mbcnt_hi(m.mask_hi, __builtin_amdgcn_mbcnt_lo(m.mask_lo, 0u)) + (hs ? 1u : 0u);
    const uint32_t row = (uint32_t)__builtin_amdgcn_ds_bpermute((int)((cnt - 1u + head_missing(m)) * 4u), (int)d.Rr);
    // its row scale (used by the last lane of each row piece)
    const float rsv = buffer_load_f1(r.rsc, row * 4u);
    __builtin_amdgcn_sched_barrier(0);
    constexpr bool EARLY = !XLDS && NB <= 2;
    if constexpr (!EARLY) {
        // (keep the multiply-adds below these loads: issued after them, the
        // loads would have only the epilogue to arrive in)
        issue_data(r, wn, mN, dN);
        __builtin_amdgcn_sched_barrier(0);
    }

    // fast decode: a whole window of one-byte varints, none continuing from
    // the window before
    const bool full = a.nbytes - b0 >= WIN_BYTES;
    const bool cont = ((d.i[0] | d.i[1] | d.i[2] | d.i[3]) & 0x80808080u) != 0u ||
                      (lane_id() == 0u && (d.ip & 0x80000000u) != 0u);
    float acc[NB];
    if (full && __ballot(cont) == 0ull)
        window_body<NB, XLDS, true>(a, r, s_x, m, d, b0, hs, wn, mN, dN, acc);
    else
        window_body<NB, XLDS, false>(a, r, s_x, m, d, b0, hs, wn, mN, dN, acc);

    // per-row pieces: segmented sums over the lanes of each row; the last
    // lane of a piece adds them to the output
    wave_seg_scan_mask<NB>(acc, S);
    const bool last = __builtin_amdgcn_inverse_ballot_w64((S >> 1) | (1ull << 63));
#pragma unroll
    for (int j = 0; j < NB; ++j) {
        const float v = a.rsc ? acc[j] * rsv : acc[j];
        const uint32_t off = (last && acc[j] != 0.0f) ? ((uint32_t)j * (uint32_t)a.out_ld + row) * 4u : OOB_OFFSET;
        __builtin_amdgcn_raw_ptr_buffer_atomic_fadd_f32(v, r.out, (int)off, 0, 0);
    }
}

// Window w of a pass with W waves: data of w + 2W and the descriptor of
// w + 3W are the loads it issues.
template <int NB, bool XLDS>
__device__ __forceinline__ void stream_step(const StreamArgs &a, const StreamRsrc &r, int64_t w, const WinMeta &m,
                                            const WinData &d, int64_t W, WinRaw &qn, WinMeta &mN, WinData &dN,
                                            const float *s_x) {
    run_window<NB, XLDS>(a, r, w, m, d, w + 2 * W, w + 3 * W, qn, mN, dN, s_x);
}

// What a window issues besides its data and descriptor loads, with no effect:
// a row-scale load (kept: marked volatile) and an atomic, both out of range.
__device__ __forceinline__ void window_dummies_load(const StreamRsrc &r) {
    (void)__builtin_amdgcn_raw_buffer_load_b32(r.rsc, (int)OOB_OFFSET, 0, (int)(1u << 31));
}
__device__ __forceinline__ void window_dummies_atomic(const StreamRsrc &r) {
    __builtin_amdgcn_raw_ptr_buffer_atomic_fadd_f32(0.0f, r.out, (int)OOB_OFFSET, 0, 0);
}

// (8 columns through the cache need more registers than 1024-thread blocks allow)
// (registers: the compiler's choice, ~100 VGPRs at one column -- capping
// them at 64 for 8 waves per SIMD measured 4 % slower on c4's layers)
template <int NB, bool XLDS>
__global__ __launch_bounds__((NB == 8 && !XLDS) ? 512 : 1024) void k_stream(StreamArgs a) {
    extern __shared__ float s_x[];
    const uint32_t nw = blockDim.x >> 6;
    const uint32_t wave = uniform(threadIdx.x >> 6);
    if constexpr (XLDS) {
        for (uint32_t i = threadIdx.x; i < (a.nx + 1u) * NB; i += blockDim.x) {
            const uint32_t c = i / NB, j = i % NB;
            s_x[i] = c == 0u ? 0.0f : (a.ent ? a.in[(c - 1u) * a.in_ld + j] * a.ent[c - 1u] : a.in[(c - 1u) * a.in_ld + j]);
        }
        __syncthreads();
    }
    const int64_t W = (int64_t)gridDim.x * nw;
    int64_t w = (int64_t)blockIdx.x * nw + wave;
    if (w >= a.nwin) return;
    StreamRsrc r;
    r.idx = buffer_rsrc(a.idx, a.nbytes + 16u);
    r.val = buffer_rsrc(a.val, a.nbytes + 16u);
    r.ner = buffer_rsrc(a.ne_row, a.n_ne * 4u);
    r.win = buffer_rsrc(a.win, (uint32_t)(a.nwin + 1) * 16u);
    r.rsc = buffer_rsrc(a.rsc ? a.rsc : a.out, a.rsc ? a.rows * 4u : 0u);
    r.out = buffer_rsrc(a.out, (uint32_t)(((int64_t)(NB - 1) * a.out_ld + a.rows) * 4));
    r.in = buffer_rsrc(a.in, XLDS ? 0u : a.nx * a.in_ld * 4u);
    r.ent = buffer_rsrc(a.ent ? a.ent : a.in, (!XLDS && a.ent) ? a.nx * 4u : 0u);
    // software pipeline over three register sets: while window w is
    // worked on, the data of the next two windows and the descriptor of the
    // one after those are in flight.  The prologue issues the same sequence
    // of memory operations as two windows of the loop (their row-scale loads
    // and atomics as no-op stand-ins), so the loop is entered with the
    // operations in flight it repeats with and the compiler's wait counts
    // stay exact throughout.
    WinRaw q;
    issue_meta(r, w, q);
    WinMeta mA = uniform_meta(q), mB, mC;
    WinData dA, dB, dC;
    issue_meta(r, w + W, q);
    window_dummies_load(r);
    issue_data(r, w, mA, dA);
    window_dummies_atomic(r);
    mB = uniform_meta(q);
    issue_meta(r, w + 2 * W, q);
    window_dummies_load(r);
    issue_data(r, w + W, mB, dB);
    window_dummies_atomic(r);
    for (;;) {
        stream_step<NB, XLDS>(a, r, w, mA, dA, W, q, mC, dC, s_x);
        w += W;
        if (w >= a.nwin) break;
        stream_step<NB, XLDS>(a, r, w, mB, dB, W, q, mA, dA, s_x);
        w += W;
        if (w >= a.nwin) break;
        stream_step<NB, XLDS>(a, r, w, mC, dC, W, q, mB, dB, s_x);
        w += W;
        if (w >= a.nwin) break;
    }
}

// Zero n floats of each of gridDim.y rows of stride ld (one launch for the
// whole batch); float4 stores when V4 (n, ld and p multiples of 4 floats).
template <bool V4>
__global__ __launch_bounds__(256) void k_fill0_rows(float *__restrict__ p, int64_t n, int64_t ld) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    float *row = p + (int64_t)blockIdx.y * ld;
    if constexpr (V4) {
        if (4 * i < n) reinterpret_cast<float4 *>(row)[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    } else {
        if (i < n) row[i] = 0.0f;
    }
}

using StreamKernel = void (*)(StreamArgs);
template <int NB>
StreamKernel stream_kernel(bool xl) {
    return xl ? k_stream<NB, true> : k_stream<NB, false>;
}
StreamKernel stream_kernel(int nb, bool xl) {
    switch (nb) {
        case 1: return stream_kernel<1>(xl);
        case 2: return stream_kernel<2>(xl);
        case 4: return stream_kernel<4>(xl);
        default: return stream_kernel<8>(xl);
    }
}

struct StreamShape {
    unsigned threads, grid;
    bool xlds;
    uint32_t lds;
};

int num_cus() {
    static const int n = [] {
        int dev = 0, v = 0;
        SILI_HIP(hipGetDevice(&dev));
        SILI_HIP(hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev));
        return v > 0 ? v : 1;
    }();
    return n;
}
int max_lds_per_block() {
    static const int n = [] {
        int dev = 0, v = 0;
        SILI_HIP(hipGetDevice(&dev));
        SILI_HIP(hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev));
        return v > 0 ? v : 65536;
    }();
    return n;
}

// Resident blocks per CU of a stream kernel at nt threads and `lds` bytes of
// dynamic LDS (cached: the occupancy query is a host computation).
int stream_occupancy(StreamKernel k, unsigned nt, uint32_t lds) {
    static std::mutex mu;
    static std::map<std::tuple<const void *, unsigned, uint32_t>, int> cache;
    std::lock_guard<std::mutex> g(mu);
    const void *f = reinterpret_cast<const void *>(k);
    const auto key = std::make_tuple(f, nt, lds);
    const auto it = cache.find(key);
    if (it != cache.end()) return it->second;
    if (lds > 65536u) (void)hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, f, (int)nt, lds) != hipSuccess) {
        (void)hipGetLastError();
        per_cu = 0;
    }
    cache[key] = per_cu;
    return per_cu;
}

constexpr int64_t STATIC_LDS = 0;  // the stream kernels' static LDS

// Launch shape for NB columns per pass: block size with the most resident
// waves per CU, a grid no larger than what is resident at once.  xmode: 0
// input through the cache, 2 input in LDS when it fits, 1 (auto) in LDS when
// it fits and staging it (input and column scale) costs at most half of a
// block's share of the stream (index + value bytes).
StreamShape stream_shape(int nb, int64_t nwin, int64_t nx, int xmode) {
    const int64_t xbytes = (nx + 1) * 4 * nb;
    const bool fits = xmode != 0 && xbytes + STATIC_LDS <= max_lds_per_block();
    StreamShape best{256, 1, false, 0};
    int best_waves = -1;
    for (const bool xl : {false, true}) {
        if (xl && !fits) continue;
        for (const unsigned nt : {256u, 512u, 1024u}) {
            if (nb == 8 && !xl && nt > 512u) continue;
            const uint32_t lds = xl ? (uint32_t)xbytes : 0u;
            const int per_cu = stream_occupancy(stream_kernel(nb, xl), nt, lds);
            if (per_cu <= 0) continue;
            const int64_t resident = (int64_t)per_cu * num_cus();
            const int64_t need = (nwin + nt / 64 - 1) / (nt / 64);
            const unsigned grid = (unsigned)std::max<int64_t>(1, std::min(resident, need));
            if (xl && xmode == 1 && 2 * xbytes * (int64_t)grid > nwin * (int64_t)WIN_BYTES) continue;
            const int waves = per_cu * (int)(nt / 64);
            // prefer XLDS when allowed, then more resident waves, then larger blocks
            const bool better = best_waves < 0 || (xl && !best.xlds) ||
                                (xl == best.xlds && waves >= best_waves);
            if (better) {
                best = StreamShape{nt, grid, xl, lds};
                best_waves = waves;
            }
        }
    }
    return best;
}

// Build d = the stream copy of s cut into K column blocks of cb columns
// (device work on L's stream; synchronous).  Sets d.failed when a block
// would not keep 31-bit offsets.
void build_stream(Layer &L, const DScatter &s, DStream &d, int K, int64_t cb) {
    hipStream_t st = L.stream;
    const int64_t rows = s.rows;
    d.valid = false;
    d.K = K;
    d.cb = cb;
    d.blocks.assign((size_t)K, DStreamBlock{});
    const int64_t n1 = rows + 1;
    DevBuf<BlkMeta> meta;
    DevBuf<uint32_t> len, pstart, ne, nepos;
    meta.ensure((size_t)K * (size_t)std::max<int64_t>(rows, 1));
    len.ensure((size_t)K * n1);
    pstart.ensure((size_t)K * n1);
    ne.ensure((size_t)K * n1);
    nepos.ensure((size_t)K * n1);
    SILI_HIP(hipMemsetAsync(meta.p, 0, sizeof(BlkMeta) * (size_t)K * (size_t)std::max<int64_t>(rows, 1), st));
    if (rows > 0)
        launch(k_spb_meta, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, st, (const uint32_t *)s.byte_start.p,
               (const uint32_t *)s.elem_start.p, (const uint8_t *)s.idx.p, rows, (uint32_t)cb, meta.p);
    launch(k_spb_len, dim3(nblk((int64_t)K * n1)), dim3(TPB), 0, st, (const BlkMeta *)meta.p, rows, K,
           (uint32_t)cb, len.p, ne.p);
    SILI_HIP(hipGetLastError());
    for (int k = 0; k < K; ++k) {
        device_exclusive_scan_u32(L, len.p + (size_t)k * n1, pstart.p + (size_t)k * n1, n1);
        device_exclusive_scan_u32(L, ne.p + (size_t)k * n1, nepos.p + (size_t)k * n1, n1);
    }
    std::vector<uint32_t> tot((size_t)K * 2);
    for (int k = 0; k < K; ++k) {
        SILI_HIP(hipMemcpyAsync(&tot[2 * (size_t)k], pstart.p + (size_t)k * n1 + rows, 4, hipMemcpyDeviceToHost, st));
        SILI_HIP(hipMemcpyAsync(&tot[2 * (size_t)k + 1], nepos.p + (size_t)k * n1 + rows, 4, hipMemcpyDeviceToHost, st));
    }
    SILI_HIP(hipStreamSynchronize(st));
    // offsets: every block starts on a window boundary; 32-bit offsets must
    // stay below 2^31 (the padded lengths were summed in 32 bits, so bound
    // them by the source first)
    if ((uint64_t)s.nbytes + 16ull * (uint64_t)rows * (uint64_t)K + (uint64_t)K * 2 * WIN_BYTES >= (1ull << 31)) {
        d.failed = true;
        return;
    }
    size_t off = 0, ne_off = 0, win_off = 0;
    for (int k = 0; k < K; ++k) {
        DStreamBlock &bk = d.blocks[(size_t)k];
        bk.nbytes = tot[2 * (size_t)k];
        bk.n_ne = tot[2 * (size_t)k + 1];
        bk.nwin = (bk.nbytes + WIN_BYTES - 1) / WIN_BYTES;
        bk.c0 = (int64_t)k * cb;
        bk.ncols = std::min<int64_t>(cb, s.cols - bk.c0);
        bk.off = off;
        bk.ne_off = ne_off;
        bk.win_off = win_off;
        off += (size_t)bk.nwin * WIN_BYTES;
        ne_off += (size_t)bk.n_ne + 1;
        win_off += (size_t)bk.nwin + 1;
    }
    d.idx.ensure(off + WIN_BYTES);
    d.val.ensure(off + WIN_BYTES);
    d.ne_row.ensure(ne_off + 1);
    d.ne_start.ensure(ne_off + 1);
    d.win.ensure(win_off + 1);
    SILI_HIP(hipMemsetAsync(d.idx.p, 0, off + WIN_BYTES, st));
    SILI_HIP(hipMemsetAsync(d.val.p, 0, off + WIN_BYTES, st));
    for (int k = 0; k < K; ++k) {
        const DStreamBlock &bk = d.blocks[(size_t)k];
        const size_t o = (size_t)k * n1;
        launch(k_sp_ne, dim3(nblk(n1)), dim3(TPB), 0, st, (const uint32_t *)ne.p + o, (const uint32_t *)nepos.p + o,
               (const uint32_t *)pstart.p + o, rows, d.ne_row.p + bk.ne_off, d.ne_start.p + bk.ne_off);
        if (rows > 0)
            launch(k_spb_copy, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, st, (const uint32_t *)s.byte_start.p,
                   (const uint8_t *)s.idx.p, (const uint8_t *)s.val.p, (const BlkMeta *)meta.p + (size_t)k * rows,
                   (const uint32_t *)pstart.p + o, rows, (uint32_t)bk.c0, d.idx.p + bk.off, d.val.p + bk.off,
                   d.win.p + bk.win_off);
        launch(k_sp_rs, dim3(nblk(bk.nwin + 1)), dim3(TPB), 0, st, (const uint32_t *)d.ne_start.p + bk.ne_off,
               bk.n_ne, bk.nwin, d.win.p + bk.win_off);
        SILI_HIP(hipGetLastError());
    }
    SILI_HIP(hipStreamSynchronize(st));
    d.valid = true;
}

// Columns per pass for a batch of B (1, 2, 4 or 8) when the input is not cut
// into column blocks: all of them when the input fits in LDS at that width,
// else the widest power of two that fits (passes re-read the stream:
// measured, B passes of one column from LDS still beat one pass of B columns
// gathered through the cache), else B in one pass through the cache.
int stream_pass_width(int64_t B, int64_t nx) {
    for (int64_t nb = B; nb >= 1; nb >>= 1)
        if ((nx + 1) * 4 * nb + STATIC_LDS <= max_lds_per_block()) return (int)nb;
    return (int)B;
}

// Column blocking for a pass of B columns: none when the input fits in LDS
// at that width (or cannot be staged at all), else the fewest equal blocks
// whose slice of the input fits.  Returns K (0: no blocking is useful).
int stream_blocks(int64_t B, int64_t cols, int64_t &cb) {
    const int64_t avail = max_lds_per_block() - STATIC_LDS;
    const int64_t cb_max = avail / (4 * B) - 1;
    if (cb_max >= cols) {
        cb = cols;
        return 1;
    }
    if (cb_max < 256) return 0;
    const int64_t K = (cols + cb_max - 1) / cb_max;
    if (K > 16) return 0;
    cb = (cols + K - 1) / K;
    return (int)K;
}

}  // namespace

bool stream_wanted(const DScatter &s, const ScaleView &sc, int64_t nb, int64_t in_ld, int skip) {
    if (!(nb == 1 || nb == 2 || nb == 4 || nb == 8) || s.nnz == 0) return false;
    // SILI_B1_STREAM (read at every call): 0 never, 1 (default) for stores of
    // at least 1 MiB of index bytes (below that one pass of the machine covers
    // the store and the segment kernels, which need no output fill, finish
    // first), 2 whenever the store allows
    const int mode = env_int("SILI_B1_STREAM", 1);
    if (mode == 0 || (mode == 1 && s.nbytes < (int64_t(1) << 20))) return false;
    if (s.stream1.failed && s.streamK.failed) return false;
    // (the kernels' buffer offsets: input and output columns in 31 bits)
    return skip == SKIP_NONE && sc.rank == 1 && in_ld == nb && s.cols + 1 < (int64_t(1) << 26) &&
           (uint64_t)s.cols * (uint64_t)nb * 4u < (1ull << 31) && (uint64_t)s.rows * (uint64_t)nb * 4u < (1ull << 31);
}

void stream_gather(Layer &L, DScatter &s, const ScaleView &sc, const float *in, int64_t B, float *out,
                   int64_t out_ld, hipStream_t st) {
    // Plan: all B columns in one pass when the input fits in LDS (whole or in
    // column blocks); else passes of fewer columns from LDS; else one pass of
    // B columns through the cache.  SILI_STREAM_XLDS=0 forces the last.
    const int force = env_int("SILI_STREAM_XLDS", -1);
    int64_t cb = s.cols;
    int K = force == 0 ? 1 : stream_blocks(B, s.cols, cb);
    int nb = (int)B;
    if (K == 0) {
        K = 1;
        cb = s.cols;
        nb = stream_pass_width(B, s.cols);
    }
    DStream *d = nullptr;
    if (K == 1) {
        d = &s.stream1;
        if (!d->valid && !d->failed) build_stream(L, s, *d, 1, s.cols);
    } else {
        d = &s.streamK;
        if (!d->valid || d->K != K || d->cb != cb) {
            d->failed = false;
            build_stream(L, s, *d, K, cb);
        }
    }
    if (!d->valid) throw_error(3, "stream copy exceeds 2 GiB");
    if (((B - 1) * out_ld + s.rows) * 4 >= (int64_t(1) << 31))
        throw_error(1, "stream_gather: output exceeds 2 GiB");
    {
        ProfScope ps("stream_zero", st);
        const bool v4 = s.rows % 4 == 0 && out_ld % 4 == 0 && (reinterpret_cast<uintptr_t>(out) & 15u) == 0;
        const int64_t per = v4 ? s.rows / 4 : s.rows;
        const dim3 grid((unsigned)((per + 255) / 256), (unsigned)B);
        if (v4) launch(k_fill0_rows<true>, grid, dim3(256), 0, st, out, s.rows, out_ld);
        else launch(k_fill0_rows<false>, grid, dim3(256), 0, st, out, s.rows, out_ld);
    }
    // input staging: off when forced, forced on when forced or when column
    // blocks (made for it) or several passes are in use, else automatic
    const int xmode = force == 0 ? 0 : (force > 0 || K > 1 || nb < B) ? 2 : 1;
    for (const DStreamBlock &bk : d->blocks) {
        if (bk.nwin == 0) continue;
        // several passes only with the input in LDS; otherwise one pass of all B
        int pnb = nb;
        StreamShape sh = stream_shape(pnb, bk.nwin, bk.ncols, xmode);
        if (pnb < B && !sh.xlds) {
            pnb = (int)B;
            sh = stream_shape(pnb, bk.nwin, bk.ncols, 0);
        }
        for (int64_t b0 = 0; b0 < B; b0 += pnb) {
            StreamArgs a{d->win.p + bk.win_off, bk.nwin, d->idx.p + bk.off, d->val.p + bk.off,
                         d->ne_row.p + bk.ne_off, (uint32_t)bk.nbytes,
                         (uint32_t)bk.n_ne, in + bk.c0 * B + b0, (uint32_t)B, sc.ent ? sc.ent + bk.c0 : nullptr,
                         sc.row, (uint32_t)bk.ncols, (uint32_t)s.rows, out + b0 * out_ld, out_ld};
            ProfScope ps(sh.xlds ? "stream_lds" : "stream", st);
            launch(stream_kernel(pnb, sh.xlds), dim3(sh.grid), dim3(sh.threads), sh.xlds ? sh.lds : 0u, st, a);
        }
    }
    SILI_HIP(hipGetLastError());
}

}  // namespace sili
