// stream.hip -- batch-1 gather split by index bytes ("stream" kernels).
//
// out[row] = sum over the row's entries of dec(code) * S(row, col) * in[col]
// for one input vector (the forward y = W x over the shadow store, or dx =
// W^T g over the canonical one; linear_disldo.hpp:68-345 / :962-1951 at batch
// 1).  The per-row segment kernels give every row its own work items, so a
// row slightly longer than a work item costs two wave passes; here the work
// is cut into fixed 512-byte windows of the concatenated index stream
// (WinDesc), so every wave pass decodes 64 x 8 index bytes whatever the row
// lengths.  Lane l of a window owns index bytes [8l, 8l + 8):
//   - rows starting inside the window are placed on the lanes holding their
//     first byte (at most one per lane: the store has no row of 1-7 bytes),
//   - the running column of each lane comes from one wave prefix sum of the
//     lanes' delta sums, restarted at row starts,
//   - per-row partial sums are combined by a segmented wave scan and leave
//     as one atomic add per row piece (the caller's output is zeroed first).
// A window whose bytes are all one-byte varints (every byte ends an entry)
// takes a decode without continuation handling; any other window (long
// deltas, the stream's partial last window) takes the general decode.
//
// XLDS: the block first stages in[c] * ent_scale[c] in LDS, so a synapse
// costs one LDS read; otherwise in and the column scale come through buffer
// loads.  The FP4 code is expanded by v_cvt_scalef32_pk_f32_fp4 (OCP E2M1:
// the reference decode for every code but 8, which never reaches these
// kernels: they serve only layers without non-finite weights, SKIP_NONE).
#include "layer.hpp"
#include "wave.hpp"

#include <algorithm>
#include <map>
#include <mutex>
#include <tuple>

namespace sili {

namespace {

constexpr uint32_t SLOT_NONE = 0xFFFFFFFFu;
constexpr uint32_t MAX_WAVES = 16;

struct StreamArgs {
    const WinDesc *win;          // nwin + 1
    int64_t nwin;
    const uint8_t *idx;
    const uint8_t *val;
    const uint32_t *byte_start;  // rows + 1
    uint32_t nbytes, nnz;
    const float *in;             // in[c], c < nx
    const float *ent;            // column scale (NULL: ones)
    const float *rsc;            // row scale (NULL: ones)
    uint32_t nx;
    float *out;                  // out[row], zeroed beforehand
};

// Registers of one window: its descriptor and the next one (whose elem and
// rs_lo bound this window's entries and rows), the lane's index bytes, the
// index dword before the window (lane 0), the lane's value dwords and one
// row start per lane.
struct WinRegs {
    WinDesc m, mn;
    uint32_t i0, i1, ip;
    uint32_t v0, v1, v2;
    uint32_t R;
};

__device__ __forceinline__ WinDesc uniform_win(const uint4 q) {
    return WinDesc{uniform(q.x), uniform(q.y), uniform(q.z), uniform(q.w)};
}
__device__ __forceinline__ uint4 load_win_raw(const WinDesc *p) { return *reinterpret_cast<const uint4 *>(p); }

__device__ __forceinline__ uint2 buffer_load_u2(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, 0));
}
__device__ __forceinline__ uint32_t buffer_load_u1(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0);
}

// Issue the loads of window w (descriptors already in r.m / r.mn).
__device__ __forceinline__ void load_window(const StreamArgs &a, int64_t w, WinRegs &r) {
    const uint32_t lane = lane_id();
    const uint32_t b0 = (uint32_t)w * WIN_BYTES;
    const uint32_t nb = min(a.nbytes - b0, WIN_BYTES);
    // index bytes (the store keeps >= 64 bytes of padding; lanes past the
    // window's end read 0, bytes at or past nb are masked by the decode)
    const uint2 iw = buffer_load_u2(buffer_rsrc(a.idx + b0, nb + 8u), 8u * lane);
    r.i0 = iw.x;
    r.i1 = iw.y;
    r.ip = (lane == 0u && b0 > 0u) ? *reinterpret_cast<const uint32_t *>(a.idx + b0 - 4u) : 0u;
    // value bytes [elem, elem + 512) from their aligned dword
    const uint32_t vbase = r.m.elem & ~3u;
    const __amdgpu_buffer_rsrc_t rv = buffer_rsrc(a.val + vbase, a.nnz - vbase + 8u);
    r.v0 = buffer_load_u1(rv, 8u * lane);
    r.v1 = buffer_load_u1(rv, 8u * lane + 4u);
    r.v2 = buffer_load_u1(rv, 8u * lane + 8u);
    // first bytes of the rows starting in the window, and of the one after
    const uint32_t nr = r.mn.rs_lo - r.m.rs_lo;
    r.R = lane <= nr ? a.byte_start[r.m.rs_lo + lane] : 0u;
}

// Weight code of value byte k (0..3) of dw: the high nibble.  The conversion
// yields both nibbles of the byte, low nibble first.
template <int K>
__device__ __forceinline__ float fp4_code_hi(uint32_t dw) {
    return __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(dw, 1.0f, K)[1];
}

template <bool XLDS, bool FAST>
__device__ __forceinline__ void run_window(const StreamArgs &a, int64_t w, const WinRegs &r, uint32_t *slot,
                                           uint32_t *vb, const float *s_x, __amdgpu_buffer_rsrc_t rin,
                                           __amdgpu_buffer_rsrc_t rent) {
    const uint32_t lane = lane_id();
    const uint32_t b0 = (uint32_t)w * WIN_BYTES;
    const uint32_t nb = min(a.nbytes - b0, WIN_BYTES);
    const uint32_t nr = r.mn.rs_lo - r.m.rs_lo;

    // rows starting in the window -> the lane holding their first byte
    slot[lane] = SLOT_NONE;
    wave_lds_sync();
    const uint32_t Rn = (uint32_t)__shfl_down((int)r.R, 1, 64);
    const uint32_t rel = r.R - b0;
    if (lane < nr && Rn > r.R && rel < WIN_BYTES) {
        slot[rel >> 3] = (lane << 3) | (rel & 7u);
    }
    wave_lds_sync();
    const uint32_t sl = slot[lane];
    const bool hs = sl != SLOT_NONE;
    const uint32_t so = hs ? (sl & 7u) : 8u;        // byte of the row start
    const uint32_t srow = r.m.rs_lo + (sl >> 3);    // the row starting there
    const uint64_t S = __ballot(hs);
    const uint64_t lt = S & ((1ull << lane) - 1ull);
    const int sp = lt ? 63 - (int)__clzll(lt) : -1;  // latest lane before this one with a row start
    const int spc = sp < 0 ? 0 : sp;
    const uint32_t hrow_s = (uint32_t)__shfl((int)srow, spc, 64);
    const uint32_t hrow = sp < 0 ? r.m.row0 : hrow_s;  // row of this lane's first bytes

    // deltas of the entries ending at each byte (0 where no entry ends)
    uint32_t dv[8];
    uint32_t tmask = 0xFFu;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        dv[i] = (r.i0 >> (8 * i)) & 0xFFu;
        dv[4 + i] = (r.i1 >> (8 * i)) & 0xFFu;
    }
    if constexpr (!FAST) {
        // the previous 4 bytes: the previous lane's, or those before the window
        const uint32_t pw0 = (uint32_t)__shfl_up((int)r.i1, 1, 64);
        const uint32_t pw = lane ? pw0 : r.ip;
        uint32_t k = 0;  // trailing continuation bytes before this lane (a varint ending here)
#pragma unroll
        for (int i = 3; i >= 0; --i) {
            const bool cont = ((pw >> (8 * i + 7)) & 1u) != 0u;
            k = (k == 3u - (uint32_t)i && cont) ? k + 1u : k;
        }
        uint32_t acc = 0, shift = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const bool use = (uint32_t)i >= 4u - k;
            acc = use ? (acc | (((pw >> (8 * i)) & 0x7Fu) << shift)) : acc;
            shift = use ? shift + 7u : shift;
        }
        tmask = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t b = dv[i];
            const bool valid = 8u * lane + (uint32_t)i < nb;
            acc |= (b & 0x7Fu) << (shift < 32u ? shift : 0u);
            const bool term = valid && (b & 0x80u) == 0u;
            dv[i] = term ? acc : 0u;
            tmask |= term ? (1u << i) : 0u;
            acc = term ? 0u : acc;
            shift = term ? 0u : shift + 7u;
        }
    }

    // column entering the lane: wave prefix of the lanes' delta sums, restarted
    // at the latest row start (a row's first delta is absolute)
    uint32_t full = 0, head = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        full += dv[i];
        head += (uint32_t)i < so ? dv[i] : 0u;
    }
    const uint32_t dsum = hs ? full - head : full;
    const uint32_t P = wave_incl_scan(dsum), Pe = P - dsum;
    const uint32_t Pe_s = (uint32_t)__shfl((int)Pe, spc, 64);
    uint32_t col = sp < 0 ? r.m.carry + Pe : Pe - Pe_s;

    // value bytes of the lane's entries, in entry order
    const uint32_t va = r.m.elem & 3u;
    const uint32_t w0 = __builtin_amdgcn_alignbyte(r.v1, r.v0, va);
    const uint32_t w1 = __builtin_amdgcn_alignbyte(r.v2, r.v1, va);
    uint32_t q0 = w0, q1 = w1;
    if constexpr (!FAST) {
        const uint32_t cnt = (uint32_t)__popc(tmask);
        const uint32_t o = wave_incl_scan(cnt) - cnt;  // entries of the window before this lane
        vb[2u * lane] = w0;
        vb[2u * lane + 1u] = w1;
        wave_lds_sync();
        const uint32_t d0 = vb[o >> 2], d1 = vb[(o >> 2) + 1u], d2 = vb[(o >> 2) + 2u];
        q0 = __builtin_amdgcn_alignbyte(d1, d0, o & 3u);
        q1 = __builtin_amdgcn_alignbyte(d2, d1, o & 3u);
    }

    // gather; the lane's sum restarts at the row start (the part before it
    // closes the previous row)
    float acc = 0.0f, hsum = 0.0f;
    uint32_t j = 0;  // entry ordinal in the lane
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        if ((uint32_t)i == so) {
            hsum = acc;
            acc = 0.0f;
            col = 0u;
        }
        col += dv[i];
        if constexpr (FAST) {
            float wq;
            switch (i & 3) {
                case 0: wq = fp4_code_hi<0>(i < 4 ? q0 : q1); break;
                case 1: wq = fp4_code_hi<1>(i < 4 ? q0 : q1); break;
                case 2: wq = fp4_code_hi<2>(i < 4 ? q0 : q1); break;
                default: wq = fp4_code_hi<3>(i < 4 ? q0 : q1); break;
            }
            float xv;
            if constexpr (XLDS) xv = s_x[col];
            else xv = buffer_load_f1(rin, col * 4u) * (a.ent ? buffer_load_f1(rent, col * 4u) : 1.0f);
            acc = __builtin_fmaf(wq, xv, acc);
        } else {
            if ((tmask >> i) & 1u) {
                const uint32_t q = (j < 4u ? q0 : q1) >> (8u * (j & 3u));
                const float wq = fp4_code_hi<0>(q);
                float xv;
                if constexpr (XLDS) xv = s_x[col];
                else xv = buffer_load_f1(rin, col * 4u) * (a.ent ? buffer_load_f1(rent, col * 4u) : 1.0f);
                acc = __builtin_fmaf(wq, xv, acc);
                ++j;
            }
        }
    }
    if constexpr (!FAST) wave_lds_sync();  // vb is rewritten by the next window

    // segmented inclusive scan of the open-row sums (segments begin at row
    // starts and at lane 0)
    const uint64_t le = S & (lane == 63u ? ~0ull : ((2ull << lane) - 1ull));
    const uint32_t dist = le ? lane - (uint32_t)(63 - (int)__clzll(le)) : lane;
    float c = acc;
#pragma unroll
    for (uint32_t d = 1; d < 64u; d <<= 1) {
        const float t = __shfl_up(c, d, 64);
        c = d <= dist ? c + t : c;
    }
    const float cin0 = __shfl_up(c, 1, 64);
    const float cin = lane ? cin0 : 0.0f;  // open-row sum entering this lane
    if (hs) {
        const float tot = cin + hsum;  // the row open before this lane's row start ends here
        if (tot != 0.0f) atomicAdd(a.out + hrow, a.rsc ? tot * a.rsc[hrow] : tot);
    }
    if (lane == 63u) {
        const uint32_t orow = hs ? srow : hrow;
        if (c != 0.0f) atomicAdd(a.out + orow, a.rsc ? c * a.rsc[orow] : c);
    }
}

template <bool XLDS>
__global__ __launch_bounds__(1024) void k_stream1(StreamArgs a) {
    extern __shared__ float s_x[];
    __shared__ uint32_t s_slot[MAX_WAVES][64];
    __shared__ uint32_t s_vb[MAX_WAVES][132];
    const uint32_t nw = blockDim.x >> 6;
    const uint32_t wave = uniform(threadIdx.x >> 6);
    if constexpr (XLDS) {
        for (uint32_t i = threadIdx.x; i < a.nx; i += blockDim.x) s_x[i] = a.ent ? a.in[i] * a.ent[i] : a.in[i];
        __syncthreads();
    }
    const int64_t W = (int64_t)gridDim.x * nw;
    int64_t w = (int64_t)blockIdx.x * nw + wave;
    if (w >= a.nwin) return;
    const __amdgpu_buffer_rsrc_t rin = buffer_rsrc(a.in, XLDS ? 0u : a.nx * 4u);
    const __amdgpu_buffer_rsrc_t rent = buffer_rsrc(a.ent ? a.ent : a.in, (!XLDS && a.ent) ? a.nx * 4u : 0u);
    uint32_t *slot = s_slot[wave];
    uint32_t *vb = s_vb[wave];
    const uint32_t lane = lane_id();
    // software pipeline: data of the next window and descriptors of the one
    // after are in flight while a window is processed
    WinRegs cur;
    cur.m = uniform_win(load_win_raw(a.win + w));
    cur.mn = uniform_win(load_win_raw(a.win + w + 1));
    load_window(a, w, cur);
    uint4 nm = make_uint4(0, 0, 0, 0), nmn = make_uint4(0, 0, 0, 0);
    if (w + W < a.nwin) {
        nm = load_win_raw(a.win + w + W);
        nmn = load_win_raw(a.win + w + W + 1);
    }
    for (; w < a.nwin; w += W) {
        WinRegs nxt = cur;
        if (w + W < a.nwin) {
            nxt.m = uniform_win(nm);
            nxt.mn = uniform_win(nmn);
            load_window(a, w + W, nxt);
            if (w + 2 * W < a.nwin) {
                nm = load_win_raw(a.win + w + 2 * W);
                nmn = load_win_raw(a.win + w + 2 * W + 1);
            }
        }
        // fast decode: a whole window of one-byte varints, none continuing
        // from the window before
        const bool full = a.nbytes - (uint32_t)w * WIN_BYTES >= WIN_BYTES;
        const bool cont = ((cur.i0 | cur.i1) & 0x80808080u) != 0u || (lane == 0u && (cur.ip & 0x80000000u) != 0u);
        if (full && __ballot(cont) == 0ull) run_window<XLDS, true>(a, w, cur, slot, vb, s_x, rin, rent);
        else run_window<XLDS, false>(a, w, cur, slot, vb, s_x, rin, rent);
        cur = nxt;
    }
}

__global__ __launch_bounds__(256) void k_fill0(float *__restrict__ p, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) p[i] = 0.0f;
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

// Resident blocks per CU of k_stream1<xl> at nt threads and `lds` bytes of
// dynamic LDS (cached: the occupancy query is a host computation).
int stream_occupancy(bool xl, unsigned nt, uint32_t lds) {
    static std::mutex mu;
    static std::map<std::tuple<bool, unsigned, uint32_t>, int> cache;
    std::lock_guard<std::mutex> g(mu);
    const auto key = std::make_tuple(xl, nt, lds);
    const auto it = cache.find(key);
    if (it != cache.end()) return it->second;
    const void *f = reinterpret_cast<const void *>(xl ? k_stream1<true> : k_stream1<false>);
    if (xl && lds > 65536u)
        (void)hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, f, (int)nt, lds) != hipSuccess) {
        (void)hipGetLastError();
        per_cu = 0;
    }
    cache[key] = per_cu;
    return per_cu;
}

// Launch shape: block size with the most resident waves per CU, a grid no
// larger than what is resident at once; XLDS when the input fits in LDS and
// staging it (input and column scale) costs at most half of a block's share
// of the stream (index + value bytes).
StreamShape stream_shape(const GatherPlan &p) {
    static const int force = env_int("SILI_STREAM_XLDS", -1);  // -1 auto, 0 off, 1 on when it fits
    const int64_t static_lds = (int64_t)MAX_WAVES * (64 + 132) * 4;
    const int64_t xbytes = p.cols * 4;
    const bool fits = xbytes + static_lds <= max_lds_per_block();
    StreamShape best{256, 1, false, 0};
    int best_waves = -1;
    for (const bool xl : {false, true}) {
        if (xl && !fits) continue;
        for (const unsigned nt : {256u, 512u, 1024u}) {
            const uint32_t lds = xl ? (uint32_t)xbytes : 0u;
            const int per_cu = stream_occupancy(xl, nt, lds);
            if (per_cu <= 0) continue;
            const int64_t resident = (int64_t)per_cu * num_cus();
            const int64_t need = (p.nwin + nt / 64 - 1) / (nt / 64);
            const unsigned grid = (unsigned)std::max<int64_t>(1, std::min(resident, need));
            if (xl) {
                const bool auto_ok = 2 * xbytes * (int64_t)grid <= p.nwin * (int64_t)WIN_BYTES;
                if (force == 0 || (force < 0 && !auto_ok)) continue;
            }
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

}  // namespace

// SILI_B1_STREAM (read at every call): 0 never, 1 (default) for stores of
// at least 2048 windows (1 MiB of index bytes: below that one pass of the
// machine covers the store and the segment kernels, which need no output
// fill, finish first), 2 whenever the store allows.
bool gather_stream_used(const GatherPlan &p, const ScaleView &sc, int64_t nb, int64_t in_ld, int skip) {
    if (nb != 1) return false;
    const int mode = env_int("SILI_B1_STREAM", 1);
    if (mode == 0 || (mode == 1 && p.nwin < 2048)) return false;
    return nb == 1 && p.stream_ok && p.nwin > 0 && skip == SKIP_NONE && sc.rank == 1 && in_ld == 1 &&
           p.cols * 4 < (int64_t(1) << 31);
}

void launch_gather_stream(const GatherPlan &p, const ScaleView &sc, const float *in, float *out, hipStream_t st) {
    {
        ProfScope ps("stream_zero", st);
        launch(k_fill0, dim3((unsigned)((p.rows + 255) / 256)), dim3(256), 0, st, out, p.rows);
    }
    StreamArgs a{p.win, p.nwin, p.idx, p.val, p.byte_start, (uint32_t)p.nbytes, (uint32_t)p.nnz,
                 in, sc.ent, sc.row, (uint32_t)p.cols, out};
    const StreamShape sh = stream_shape(p);
    if (sh.xlds) {
        ProfScope ps("stream_lds", st);
        launch(k_stream1<true>, dim3(sh.grid), dim3(sh.threads), sh.lds, st, a);
    } else {
        ProfScope ps("stream", st);
        launch(k_stream1<false>, dim3(sh.grid), dim3(sh.threads), 0u, st, a);
    }
    SILI_HIP(hipGetLastError());
}

}  // namespace sili
