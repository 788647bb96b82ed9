// patch.hip -- row patches of the compact stores, for the reference's
// synaptogenesis policy (delta_csr_synap_row_step, delta_csr_memory.hpp:
// 1021-1264, which edits one row of its store in place).
//
// A policy call changes one block row of the canonical layout (the edited
// row, the rows a demotion or promotion moves slots between, the block row's
// tiles) and, through them, a few rows of each shadow.  Instead of decoding,
// sorting and re-encoding both stores, a patch:
//   1. stages the rows it rewrites from the device into pinned host memory
//      (one kernel per store orientation, one sync for all of them);
//   2. encodes the new rows on the host exactly as the device encoder would
//      (ULEB128 deltas, work items of <= seg_len index bytes);
//   3. writes every array anew into its second buffer in one launch: runs of
//      unchanged rows copied with their starts, work items and permutation
//      values shifted by the rows' size changes before them, the new rows from
//      the uploaded patch content; then the buffers swap.
// The result is the structure a full rebuild of the same synapse set gives
// (the build is a pure function of the set), at the cost of one pass over
// the arrays' bytes.
#include "../../include/sili_hip.h"
#include "layer.hpp"

#include <algorithm>
#include <cstring>
#include <map>
#include <set>
#include <vector>

#include <rocprim/rocprim.hpp>

namespace sili {

namespace {

constexpr unsigned TPB = 256;
inline unsigned nblk(int64_t n) { return (unsigned)((n + TPB - 1) / TPB); }

// ---- staging ---------------------------------------------------------------
// One store orientation's rows into pinned memory, as 32-bit words:
// out[0] = words needed; per row 6 header words (b0, b1, e0, e1, slo, shi);
// then per row its payload: index bytes, element bytes (elem_bytes each),
// flag bytes (flags != NULL), each padded to whole words, then permutation
// words (perm != NULL).  Nothing past the header is written when the
// payload does not fit `cap` words.  Up to STAGE_INLINE row numbers travel
// in the arguments; longer lists in device memory (rows).
constexpr uint32_t STAGE_MAX_ROWS = 4096, STAGE_INLINE = 192, STAGE_TPB = 1024;
struct StageArgs {
    const uint32_t *bstart, *estart;
    const uint8_t *idx, *elems, *flags;
    const uint32_t *perm;
    const SegDesc *seg;
    uint32_t nseg, elem_bytes, m, nrows;
    const uint32_t *rows;
    uint32_t *out;
    uint64_t cap;
    uint32_t inl[STAGE_INLINE];
};

// First work item of a row >= `row` (items ordered by row), by a galloping
// search from item `g` (a row's items start near row * nseg / rows), then
// bisection: a few dependent loads instead of log2(nseg).
__device__ __forceinline__ uint32_t seg_lower(const SegDesc *seg, uint32_t n, uint32_t row, uint32_t g) {
    uint32_t lo = 0, hi = n;  // the answer lies in [lo, hi]
    if (g < n) {
        uint32_t s = 1;
        if (seg[g].row >= row) {
            hi = g;
            while (true) {
                if (hi < s) { lo = 0; break; }
                const uint32_t p = hi - s;
                if (seg[p].row < row) { lo = p + 1; break; }
                hi = p;
                s <<= 1;
            }
        } else {
            lo = g + 1;
            while (true) {
                const uint64_t p = (uint64_t)lo + s - 1;
                if (p >= n) { hi = n; break; }
                if (seg[p].row >= row) { hi = (uint32_t)p; break; }
                lo = (uint32_t)p + 1;
                s <<= 1;
            }
        }
    }
    while (lo < hi) {
        const uint32_t mid = (lo + hi) >> 1;
        if (seg[mid].row < row) lo = mid + 1;
        else hi = mid;
    }
    return lo;
}
__device__ __forceinline__ uint32_t pack4(const uint8_t *p, uint64_t i, uint64_t end) {
    uint32_t w = 0;
    for (uint32_t k = 0; k < 4u; ++k)
        if (i + k < end) w |= (uint32_t)p[i + k] << (8u * k);
    return w;
}
__device__ __forceinline__ uint32_t words_of(uint64_t bytes) { return (uint32_t)((bytes + 3u) / 4u); }

// Rows in parallel: each thread sizes up to 4 consecutive rows, a block
// scan places them, then each wave copies whole rows.
__global__ __launch_bounds__(STAGE_TPB) void k_stage_rows(StageArgs a) {
    __shared__ uint32_t s_off[STAGE_MAX_ROWS + 1];
    __shared__ uint32_t s_wave[STAGE_TPB / 64];
    const uint32_t t = threadIdx.x, lane = t & 63u, wave = t >> 6;
    const uint32_t per = (a.m + STAGE_TPB - 1) / STAGE_TPB;  // rows per thread (<= 4)
    uint32_t mine = 0;
    for (uint32_t k = 0; k < per; ++k) {
        const uint32_t j = t * per + k;
        if (j >= a.m) break;
        const uint32_t r = a.m <= STAGE_INLINE ? a.inl[j] : a.rows[j];
        const uint32_t b0 = a.bstart[r], b1 = a.bstart[r + 1], e0 = a.estart[r], e1 = a.estart[r + 1];
        uint32_t *h = a.out + 1u + 6u * j;
        h[0] = b0;
        h[1] = b1;
        h[2] = e0;
        h[3] = e1;
        const uint32_t g = (uint32_t)((uint64_t)r * a.nseg / max(a.nrows, 1u));
        h[4] = seg_lower(a.seg, a.nseg, r, g);
        h[5] = seg_lower(a.seg, a.nseg, r + 1u, h[4]);
        const uint32_t ne = e1 - e0;
        const uint32_t w = words_of(b1 - b0) + words_of((uint64_t)ne * a.elem_bytes) + (a.flags ? words_of(ne) : 0u) +
                           (a.perm ? ne : 0u);
        s_off[j] = w;
        mine += w;
    }
    // exclusive scan of the threads' totals
    uint32_t incl = mine;
    for (uint32_t o = 1; o < 64u; o <<= 1) {
        const uint32_t y = __shfl_up(incl, o, 64);
        if (lane >= o) incl += y;
    }
    if (lane == 63u) s_wave[wave] = incl;
    __syncthreads();
    uint32_t before = 0, total = 0;
    for (uint32_t w = 0; w < STAGE_TPB / 64u; ++w) {
        const uint32_t v = s_wave[w];
        before += w < wave ? v : 0u;
        total += v;
    }
    uint32_t run = before + incl - mine;
    for (uint32_t k = 0; k < per; ++k) {
        const uint32_t j = t * per + k;
        if (j >= a.m) break;
        const uint32_t w = s_off[j];
        s_off[j] = run;
        run += w;
    }
    if (t == 0) a.out[0] = 1u + 6u * a.m + total;
    __syncthreads();
    if ((uint64_t)1u + 6u * a.m + total > a.cap) return;
    uint32_t *pay = a.out + 1u + 6u * a.m;
    for (uint32_t j = wave; j < a.m; j += STAGE_TPB / 64u) {
        const uint32_t r = a.m <= STAGE_INLINE ? a.inl[j] : a.rows[j];
        const uint32_t b0 = a.bstart[r], b1 = a.bstart[r + 1], e0 = a.estart[r], e1 = a.estart[r + 1];
        const uint32_t ne = e1 - e0;
        uint32_t *o = pay + s_off[j];
        const uint32_t wi = words_of(b1 - b0);
        for (uint32_t w = lane; w < wi; w += 64u) o[w] = pack4(a.idx, (uint64_t)b0 + 4u * w, b1);
        o += wi;
        const uint64_t eb0 = (uint64_t)e0 * a.elem_bytes, eb1 = (uint64_t)e1 * a.elem_bytes;
        const uint32_t we = words_of(eb1 - eb0);
        for (uint32_t w = lane; w < we; w += 64u) o[w] = pack4(a.elems, eb0 + 4u * w, eb1);
        o += we;
        if (a.flags) {
            const uint32_t wf = words_of(ne);
            for (uint32_t w = lane; w < wf; w += 64u) o[w] = pack4(a.flags, (uint64_t)e0 + 4u * w, e1);
            o += wf;
        }
        if (a.perm)
            for (uint32_t k = lane; k < ne; k += 64u) o[k] = a.perm[e0 + k];
    }
}

// The activity accumulators (acc_in then acc_grad) into pinned memory.
__global__ void k_stage_acc(const float *__restrict__ a, int64_t na, const float *__restrict__ b, int64_t nb,
                            float *__restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i < na) out[i] = a[i];
    else if (i < na + nb) out[i] = b[i - na];
}

// ---- the patch kernel --------------------------------------------------------
// Each piece writes n elements at dst: copied from src (mode 0: bytes; 1:
// u32 + add0; 2: u32 remapped; 3: work items with add0 on their byte
// offsets and add1 on their element offsets).  Blocks take chunks of the
// pieces in order (chunk0: the piece's first block).
enum : uint32_t { PM_BYTES = 0, PM_U32_ADD = 1, PM_U32_REMAP = 2, PM_SEG = 3 };
struct alignas(16) PatchPiece {
    uint64_t src, dst, n;
    uint32_t mode, chunk0;
    int64_t add0, add1;
    uint64_t aux;  // PM_U32_REMAP: device address of its Remap
    uint64_t pad;
};
// v -> v (v < lo), map[v - lo] (lo <= v < hi), v + delta (v >= hi)
struct alignas(16) Remap {
    uint64_t lo, hi;
    int64_t delta;
    uint64_t map;  // device address of (hi - lo) u32
};
__host__ __device__ constexpr uint32_t chunk_elems(uint32_t mode) {
    return mode == PM_BYTES ? 8192u : mode == PM_SEG ? 512u : 2048u;
}

__global__ __launch_bounds__(TPB) void k_patch_apply(const PatchPiece *__restrict__ pc, uint32_t np) {
    const uint32_t b = blockIdx.x;
    uint32_t lo = 0, hi = np;  // last piece with chunk0 <= b
    while (hi - lo > 1u) {
        const uint32_t mid = (lo + hi) >> 1;
        if (pc[mid].chunk0 <= b) lo = mid;
        else hi = mid;
    }
    const PatchPiece P = pc[lo];
    const uint32_t ce = chunk_elems(P.mode);
    const uint64_t base = (uint64_t)(b - P.chunk0) * ce;
    const uint64_t end = min<uint64_t>(P.n, base + ce);
    if (P.mode == PM_BYTES) {
        // whole aligned destination words from two aligned source words each
        // (v_alignbyte); the bytes of partial words at the chunk's ends one by
        // one (neighbouring pieces own the rest of those words)
        const uint8_t *s = reinterpret_cast<const uint8_t *>(P.src);
        uint8_t *d = reinterpret_cast<uint8_t *>(P.dst);
        const uint64_t dlo = P.dst + base, dhi = P.dst + end;
        const uint64_t wlo = (dlo + 3u) & ~uint64_t(3), whi = dhi & ~uint64_t(3);
        if (wlo >= whi) {
            for (uint64_t i = base + threadIdx.x; i < end; i += TPB) d[i] = s[i];
        } else {
            const uint64_t head = wlo - dlo, tail = dhi - whi;
            if (threadIdx.x < head) d[base + threadIdx.x] = s[base + threadIdx.x];
            if (threadIdx.x < tail) d[(whi - P.dst) + threadIdx.x] = s[(whi - P.dst) + threadIdx.x];
            const uint64_t nw = (whi - wlo) / 4u;
            const uint64_t s0 = P.src + (wlo - P.dst);  // source address of the first whole word
            const uint32_t k = (uint32_t)(s0 & 3u);
            const uint32_t *sw = reinterpret_cast<const uint32_t *>(s0 & ~uint64_t(3));
            uint32_t *dw = reinterpret_cast<uint32_t *>(wlo);
            if (k == 0u) {
                for (uint64_t i = threadIdx.x; i < nw; i += TPB) dw[i] = sw[i];
            } else {
                for (uint64_t i = threadIdx.x; i < nw; i += TPB)
                    dw[i] = __builtin_amdgcn_alignbyte(sw[i + 1], sw[i], k);
            }
        }
    } else if (P.mode == PM_U32_ADD) {
        const uint32_t *s = reinterpret_cast<const uint32_t *>(P.src);
        uint32_t *d = reinterpret_cast<uint32_t *>(P.dst);
        for (uint64_t i = base + threadIdx.x; i < end; i += TPB) d[i] = (uint32_t)((int64_t)s[i] + P.add0);
    } else if (P.mode == PM_U32_REMAP) {
        const uint32_t *s = reinterpret_cast<const uint32_t *>(P.src);
        uint32_t *d = reinterpret_cast<uint32_t *>(P.dst);
        const Remap R = *reinterpret_cast<const Remap *>(P.aux);
        const uint32_t *map = reinterpret_cast<const uint32_t *>(R.map);
        for (uint64_t i = base + threadIdx.x; i < end; i += TPB) {
            const uint64_t v = s[i];
            d[i] = v < R.lo ? (uint32_t)v : v >= R.hi ? (uint32_t)((int64_t)v + R.delta) : map[v - R.lo];
        }
    } else {
        const SegDesc *s = reinterpret_cast<const SegDesc *>(P.src);
        SegDesc *d = reinterpret_cast<SegDesc *>(P.dst);
        for (uint64_t i = base + threadIdx.x; i < end; i += TPB) {
            SegDesc g = s[i];
            g.byte_begin = (uint32_t)((int64_t)g.byte_begin + P.add0);
            g.byte_end = (uint32_t)((int64_t)g.byte_end + P.add0);
            g.elem_begin = (uint32_t)((int64_t)g.elem_begin + P.add1);
            g.elem_end = (uint32_t)((int64_t)g.elem_end + P.add1);
            d[i] = g;
        }
    }
}

// Rows with more than one work item (split) from a store's work items.
__global__ void k_split_from_segs(const SegDesc *__restrict__ seg, int64_t nseg, uint32_t *__restrict__ flag) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i < nseg && (seg[i].split & SEG_SPLIT) && (seg[i].split & SEG_FIRST)) flag[seg[i].row] = 1u;
}
__global__ void k_fill0_u32(uint32_t *__restrict__ p, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i < n) p[i] = 0u;
}
__global__ void k_list_rows(const uint32_t *__restrict__ flag, const uint32_t *__restrict__ pos, int64_t rows,
                            uint32_t *__restrict__ list) {
    const int64_t r = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (r < rows && flag[r]) list[pos[r]] = (uint32_t)r;
}

// ---- host encoding (the device encoder's rules, build.hip) ------------------
void uleb_put(std::vector<uint8_t> &out, uint32_t v) {
    do {
        uint8_t b = v & 0x7Fu;
        v >>= 7;
        if (v) b |= 0x80u;
        out.push_back(b);
    } while (v);
}

// Index bytes of a row (first delta from 0) and each entry's byte offset
// in the row.
void encode_row(const std::vector<uint32_t> &cols, std::vector<uint8_t> &bytes, std::vector<uint32_t> &posrel) {
    bytes.clear();
    posrel.clear();
    uint32_t prev = 0;
    for (uint32_t c : cols) {
        posrel.push_back((uint32_t)bytes.size());
        uleb_put(bytes, c - prev);
        prev = c;
    }
}

// The row's work items (k_seg_write): item j holds the entries whose varint
// starts at row offset [j*W, (j+1)*W), W = seg_bytes - 4.
void row_segs(uint32_t row, const std::vector<uint32_t> &cols, const std::vector<uint32_t> &posrel, uint32_t rb0,
              uint32_t rb1, uint32_t re0, uint32_t seg_bytes, bool emit_empty, std::vector<SegDesc> &out) {
    const uint32_t n = (uint32_t)cols.size(), W = seg_bytes - 4u;
    const uint32_t cnt = n == 0 ? (emit_empty ? 1u : 0u) : posrel[n - 1] / W + 1u;
    uint32_t eb = 0;
    for (uint32_t j = 0; j < cnt; ++j) {
        const bool last = j + 1u == cnt;
        uint32_t ee = n;
        if (!last) {
            ee = eb;
            while (ee < n && posrel[ee] < (j + 1u) * W) ++ee;
        }
        SegDesc d;
        d.row = row;
        d.elem_begin = re0 + eb;
        d.elem_end = re0 + ee;
        d.byte_begin = j == 0 ? rb0 : rb0 + posrel[eb];
        d.byte_end = last ? rb1 : rb0 + posrel[ee];
        d.base_col = eb > 0 ? cols[eb - 1] : 0u;
        d.split = (cnt > 1u ? SEG_SPLIT : 0u) | (j == 0 ? SEG_FIRST : 0u);
        d.pad1 = 0u;
        out.push_back(d);
        eb = ee;
    }
}

// A row's new content for one store orientation.
struct NewRow {
    uint32_t row = 0;
    std::vector<uint32_t> cols;
    std::vector<uint8_t> elems;  // elem_bytes per entry
    std::vector<uint8_t> flags;  // per entry (flagged stores)
    std::vector<uint32_t> perm;  // per entry (permuted stores)
};

// The views of one store orientation's arrays that a patch rewrites.
struct StoreArrays {
    DevBuf<uint32_t> *bstart, *estart;
    DevBuf<uint8_t> *idx, *elems, *flags;  // flags: NULL unless the store keeps them
    DevBuf<uint32_t> *perm;                // NULL unless kept
    DevBuf<SegDesc> *seg;
    DevBuf<uint32_t> *sp_bstart, *sp_estart;
    DevBuf<uint8_t> *sp_idx, *sp_elems, *sp_flags;
    DevBuf<uint32_t> *sp_perm;
    DevBuf<SegDesc> *sp_seg;
    int64_t rows, nbytes, nelems, nseg;
    uint32_t elem_bytes, seg_bytes;
    bool emit_empty;
};

// Collects the pieces of one launch and the content they copy from.
struct PatchBuilder {
    std::vector<uint8_t> blob;     // new content, 16-byte aligned parts
    struct HostPiece {
        PatchPiece p;
        bool src_blob, aux_blob;
    };
    std::vector<HostPiece> pieces;
    size_t put(const void *data, size_t bytes) {
        const size_t off = (blob.size() + 15) & ~size_t(15);
        blob.resize(off + bytes);
        if (bytes) std::memcpy(blob.data() + off, data, bytes);
        return off;
    }
    void piece(uint32_t mode, uint64_t src, bool src_blob, void *dst, uint64_t n, int64_t add0 = 0, int64_t add1 = 0,
               uint64_t aux = 0, bool aux_blob = false) {
        if (n == 0) return;
        HostPiece h{};
        h.p.src = src;
        h.p.dst = reinterpret_cast<uint64_t>(dst);
        h.p.n = n;
        h.p.mode = mode;
        h.p.add0 = add0;
        h.p.add1 = add1;
        h.p.aux = aux;
        h.src_blob = src_blob;
        h.aux_blob = aux_blob;
        pieces.push_back(h);
    }
};

// What a store orientation's patch changed, for the layer's bookkeeping.
struct StoreDelta {
    int64_t dbytes = 0, delems = 0, dseg = 0, dempty = 0;
    bool split_maybe_changed = false;
};

// Pieces rewriting store `A` with rows `edit` (ascending) replaced by `nu`
// (same order); `old[j]` is row edit[j] as staged.  Unchanged permutation
// runs are remapped through `remap` (blob offset of a Remap; ~0: add 0).
StoreDelta plan_store(PatchBuilder &P, StoreArrays &A, const std::vector<StagedRow> &old,
                      const std::vector<NewRow> &nu, uint64_t remap_off) {
    StoreDelta D;
    const size_t m = nu.size();
    // new encodings and their sizes
    std::vector<std::vector<uint8_t>> nbytes(m);
    std::vector<std::vector<uint32_t>> nposrel(m);
    int64_t tb = 0, te = 0;
    for (size_t j = 0; j < m; ++j) {
        encode_row(nu[j].cols, nbytes[j], nposrel[j]);
        tb += (int64_t)nbytes[j].size() - (int64_t)(old[j].b1 - old[j].b0);
        te += (int64_t)nu[j].cols.size() - (int64_t)(old[j].e1 - old[j].e0);
    }
    const int64_t new_bytes = A.nbytes + tb, new_elems = A.nelems + te;
    // second buffers sized for the new arrays (the work items' by the caller,
    // before any piece points into them)
    A.sp_idx->ensure((size_t)new_bytes + 64);
    A.sp_elems->ensure((size_t)new_elems * A.elem_bytes + 64);
    if (A.flags) A.sp_flags->ensure((size_t)new_elems + 64);
    if (A.perm) A.sp_perm->ensure((size_t)new_elems + 1);
    A.sp_bstart->ensure((size_t)A.rows + 1);
    A.sp_estart->ensure((size_t)A.rows + 1);
    // rows: runs of unchanged rows between the edited ones, shifted by the
    // size changes before them
    int64_t db = 0, de = 0, ds = 0;
    uint32_t pb = 0, pe = 0, ps = 0, pr = 0;  // old positions after the previous edited row; next row
    std::vector<std::vector<SegDesc>> nsegs(m);
    for (size_t j = 0; j < m; ++j) {
        const StagedRow &o = old[j];
        const uint32_t nb0 = (uint32_t)(o.b0 + db), ne0 = (uint32_t)(o.e0 + de);
        row_segs(nu[j].row, nu[j].cols, nposrel[j], nb0, nb0 + (uint32_t)nbytes[j].size(), ne0, A.seg_bytes,
                 A.emit_empty, nsegs[j]);
        const uint32_t old_cnt = o.shi - o.slo, new_cnt = (uint32_t)nsegs[j].size();
        if (old_cnt > 1 || new_cnt > 1) D.split_maybe_changed = true;
        D.dempty += (nu[j].cols.empty() ? 1 : 0) - (o.e1 == o.e0 ? 1 : 0);
        // unchanged run before this row
        P.piece(PM_BYTES, reinterpret_cast<uint64_t>(A.idx->p) + pb, false, A.sp_idx->p + pb + db, o.b0 - pb);
        P.piece(PM_BYTES, reinterpret_cast<uint64_t>(A.elems->p) + (uint64_t)pe * A.elem_bytes, false,
                A.sp_elems->p + (uint64_t)(pe + de) * A.elem_bytes, (uint64_t)(o.e0 - pe) * A.elem_bytes);
        if (A.flags)
            P.piece(PM_BYTES, reinterpret_cast<uint64_t>(A.flags->p) + pe, false, A.sp_flags->p + pe + de, o.e0 - pe);
        if (A.perm) {
            if (remap_off != ~0ull)
                P.piece(PM_U32_REMAP, reinterpret_cast<uint64_t>(A.perm->p + pe), false, A.sp_perm->p + pe + de,
                        o.e0 - pe, 0, 0, remap_off, true);
            else
                P.piece(PM_U32_ADD, reinterpret_cast<uint64_t>(A.perm->p + pe), false, A.sp_perm->p + pe + de,
                        o.e0 - pe);
        }
        P.piece(PM_SEG, reinterpret_cast<uint64_t>(A.seg->p + ps), false, A.sp_seg->p + ps + ds, o.slo - ps, db, de);
        // starts of rows (pr, row] keep their offsets shifted by the changes before
        P.piece(PM_U32_ADD, reinterpret_cast<uint64_t>(A.bstart->p + pr), false, A.sp_bstart->p + pr,
                nu[j].row + 1 - pr, db);
        P.piece(PM_U32_ADD, reinterpret_cast<uint64_t>(A.estart->p + pr), false, A.sp_estart->p + pr,
                nu[j].row + 1 - pr, de);
        // the edited row from the blob
        if (!nbytes[j].empty())
            P.piece(PM_BYTES, P.put(nbytes[j].data(), nbytes[j].size()), true, A.sp_idx->p + nb0, nbytes[j].size());
        if (!nu[j].elems.empty())
            P.piece(PM_BYTES, P.put(nu[j].elems.data(), nu[j].elems.size()), true,
                    A.sp_elems->p + (uint64_t)ne0 * A.elem_bytes, nu[j].elems.size());
        if (A.flags && !nu[j].flags.empty())
            P.piece(PM_BYTES, P.put(nu[j].flags.data(), nu[j].flags.size()), true, A.sp_flags->p + ne0,
                    nu[j].flags.size());
        if (A.perm && !nu[j].perm.empty())
            P.piece(PM_U32_ADD, P.put(nu[j].perm.data(), nu[j].perm.size() * 4), true, A.sp_perm->p + ne0,
                    nu[j].perm.size());
        if (!nsegs[j].empty())
            P.piece(PM_SEG, P.put(nsegs[j].data(), nsegs[j].size() * sizeof(SegDesc)), true,
                    A.sp_seg->p + ps + ds + (o.slo - ps), nsegs[j].size());
        db += (int64_t)nbytes[j].size() - (int64_t)(o.b1 - o.b0);
        de += (int64_t)nu[j].cols.size() - (int64_t)(o.e1 - o.e0);
        ds += (int64_t)nsegs[j].size() - (int64_t)(o.shi - o.slo);
        pb = o.b1;
        pe = o.e1;
        ps = o.shi;
        pr = nu[j].row + 1;
    }
    // the run after the last edited row
    P.piece(PM_BYTES, reinterpret_cast<uint64_t>(A.idx->p) + pb, false, A.sp_idx->p + pb + db, A.nbytes - pb);
    P.piece(PM_BYTES, reinterpret_cast<uint64_t>(A.elems->p) + (uint64_t)pe * A.elem_bytes, false,
            A.sp_elems->p + (uint64_t)(pe + de) * A.elem_bytes, (uint64_t)(A.nelems - pe) * A.elem_bytes);
    if (A.flags)
        P.piece(PM_BYTES, reinterpret_cast<uint64_t>(A.flags->p) + pe, false, A.sp_flags->p + pe + de, A.nelems - pe);
    if (A.perm) {
        if (remap_off != ~0ull)
            P.piece(PM_U32_REMAP, reinterpret_cast<uint64_t>(A.perm->p + pe), false, A.sp_perm->p + pe + de,
                    A.nelems - pe, 0, 0, remap_off, true);
        else
            P.piece(PM_U32_ADD, reinterpret_cast<uint64_t>(A.perm->p + pe), false, A.sp_perm->p + pe + de,
                    A.nelems - pe);
    }
    P.piece(PM_SEG, reinterpret_cast<uint64_t>(A.seg->p + ps), false, A.sp_seg->p + ps + ds, A.nseg - ps, db, de);
    P.piece(PM_U32_ADD, reinterpret_cast<uint64_t>(A.bstart->p + pr), false, A.sp_bstart->p + pr, A.rows + 1 - pr, db);
    P.piece(PM_U32_ADD, reinterpret_cast<uint64_t>(A.estart->p + pr), false, A.sp_estart->p + pr, A.rows + 1 - pr, de);
    D.dbytes = db;
    D.delems = de;
    D.dseg = ds;
    return D;
}

}  // namespace

// ---- staging ---------------------------------------------------------------
void stage_rows(Layer &L, const std::vector<StageReq *> &reqs) {
    hipStream_t st = L.stream;
    size_t nrows = 0;
    for (auto *q : reqs) {
        if (q->rows.size() > STAGE_MAX_ROWS) throw_error(SILI_ERR_RANGE, "stage_rows: too many rows");
        nrows += q->rows.size();
    }
    // row lists beyond STAGE_INLINE to the device (one copy), output
    // regions in pinned memory
    std::vector<size_t> cap(reqs.size(), 0), out_off(reqs.size(), 0);
    for (int attempt = 0; attempt < 2; ++attempt) {
        size_t k = 0;
        std::vector<size_t> row_off(reqs.size());
        for (size_t i = 0; i < reqs.size(); ++i) {
            row_off[i] = k;
            if (reqs[i]->rows.size() > STAGE_INLINE) k += reqs[i]->rows.size();
        }
        TmpBuf<uint32_t> drows(L, SILI_TMPKEY(drows));
        if (k) {
            L.pin_rows.ensure(k * 4);
            uint32_t *rl = reinterpret_cast<uint32_t *>(L.pin_rows.h);
            for (size_t i = 0; i < reqs.size(); ++i)
                if (reqs[i]->rows.size() > STAGE_INLINE)
                    std::copy(reqs[i]->rows.begin(), reqs[i]->rows.end(), rl + row_off[i]);
            drows.ensure(k);
            SILI_HIP(hipMemcpyAsync(drows.p, rl, k * 4, hipMemcpyHostToDevice, st));
        }
        size_t total = 0;
        for (size_t i = 0; i < reqs.size(); ++i) {
            if (cap[i] == 0) {
                // twice the store's average row, in words, plus headers
                const StageReq &q = *reqs[i];
                const double rows = (double)std::max<int64_t>(1, q.s ? q.s->rows : q.b->brows);
                const double nb = (double)(q.s ? q.s->nbytes : q.b->nbytes) / rows;
                const double ne = (double)(q.s ? q.s->nnz : q.b->ntiles) / rows;
                const double per_row = (nb + ne * (q.s ? 1.0 : 16.0) + (q.flags ? ne : 0.0) + (q.perm ? 4 * ne : 0.0)) / 4;
                cap[i] = 1 + 6 * q.rows.size() + (size_t)(2.0 * per_row * (double)q.rows.size()) + 4 * q.rows.size() + 1024;
            }
            out_off[i] = total;
            total += cap[i];
        }
        L.pin_stage.ensure(total * 4);
        uint32_t *out = reinterpret_cast<uint32_t *>(L.pin_stage.h);
        for (size_t i = 0; i < reqs.size(); ++i) {
            StageReq &q = *reqs[i];
            StageArgs a{};
            if (q.s) {
                a.bstart = q.s->byte_start.p;
                a.estart = q.s->elem_start.p;
                a.idx = q.s->idx.p;
                a.elems = q.s->val.p;
                a.seg = q.s->seg.p;
                a.nseg = (uint32_t)q.s->nseg;
                a.nrows = (uint32_t)q.s->rows;
                a.elem_bytes = 1;
            } else {
                a.bstart = q.b->byte_start.p;
                a.estart = q.b->tile_start.p;
                a.idx = q.b->idx.p;
                a.elems = q.b->tiles.p;
                a.seg = q.b->seg.p;
                a.nseg = (uint32_t)q.b->nseg;
                a.nrows = (uint32_t)q.b->brows;
                a.elem_bytes = 16;
            }
            a.flags = q.flags;
            a.perm = q.perm;
            a.m = (uint32_t)q.rows.size();
            if (a.m <= STAGE_INLINE) std::copy(q.rows.begin(), q.rows.end(), a.inl);
            else a.rows = drows.p + row_off[i];
            a.out = out + out_off[i];
            a.cap = cap[i];
            out[out_off[i]] = 0;
            if (a.m) launch(k_stage_rows, dim3(1), dim3(STAGE_TPB), 0, st, a);
        }
        SILI_HIP(hipGetLastError());
        SILI_HIP(hipStreamSynchronize(st));
        bool again = false;
        for (size_t i = 0; i < reqs.size(); ++i) {
            const uint32_t need = reqs[i]->rows.empty() ? 0u : out[out_off[i]];
            if (need > cap[i]) {
                cap[i] = need;
                again = true;
            }
        }
        if (again) {
            if (attempt == 1) throw_error(SILI_ERR_RUNTIME, "stage_rows: staging did not fit");
            continue;
        }
        for (size_t i = 0; i < reqs.size(); ++i) {
            StageReq &q = *reqs[i];
            const uint32_t eb = q.s ? 1u : 16u;
            const uint32_t *o = out + out_off[i];
            const size_t m = q.rows.size();
            q.out.assign(m, StagedRow{});
            const uint32_t *pay = o + 1 + 6 * m;
            size_t w = 0;
            for (size_t j = 0; j < m; ++j) {
                StagedRow &R = q.out[j];
                const uint32_t *h = o + 1 + 6 * j;
                R.row = q.rows[j];
                R.b0 = h[0];
                R.b1 = h[1];
                R.e0 = h[2];
                R.e1 = h[3];
                R.slo = h[4];
                R.shi = h[5];
                const uint32_t nb = R.b1 - R.b0, ne = R.e1 - R.e0;
                const uint8_t *pb = reinterpret_cast<const uint8_t *>(pay + w);
                R.idx.assign(pb, pb + nb);
                w += (nb + 3) / 4;
                const uint8_t *pe = reinterpret_cast<const uint8_t *>(pay + w);
                R.elems.assign(pe, pe + (size_t)ne * eb);
                w += ((size_t)ne * eb + 3) / 4;
                if (q.flags) {
                    const uint8_t *pf = reinterpret_cast<const uint8_t *>(pay + w);
                    R.flags.assign(pf, pf + ne);
                    w += (ne + 3) / 4;
                }
                if (q.perm) {
                    R.perm.assign(pay + w, pay + w + ne);
                    w += ne;
                }
            }
        }
        return;
    }
}

const float *stage_accumulators(Layer &L) {
    const int64_t n = L.n_in + L.n_out;
    if (L.acc_epoch == L.policy_epoch) return reinterpret_cast<const float *>(L.pin_acc.h);
    L.pin_acc.ensure((size_t)n * 4 + 4);
    if (n > 0)
        launch(k_stage_acc, dim3(nblk(n)), dim3(TPB), 0, L.stream, (const float *)L.acc_in.p, L.n_in,
               (const float *)L.acc_grad.p, L.n_out, reinterpret_cast<float *>(L.pin_acc.h));
    SILI_HIP(hipGetLastError());
    SILI_HIP(hipStreamSynchronize(L.stream));
    L.acc_epoch = L.policy_epoch;
    L.sel_in_k = L.sel_out_k = -1;
    return reinterpret_cast<const float *>(L.pin_acc.h);
}

std::vector<uint32_t> staged_cols(const StagedRow &r) {
    std::vector<uint32_t> cols;
    cols.reserve(r.e1 - r.e0);
    size_t pos = 0;
    uint32_t c = 0;
    for (uint32_t e = r.e0; e < r.e1; ++e) {
        uint32_t v = 0;
        for (uint32_t sh = 0;; sh += 7) {
            const uint8_t b = r.idx[pos++];
            v |= (uint32_t)(b & 0x7Fu) << sh;
            if (!(b & 0x80u)) break;
        }
        c += v;
        cols.push_back(c);
    }
    return cols;
}

// ---- the block-row patch -----------------------------------------------------
namespace {

inline uint8_t requant(uint32_t code) { return code == 8u ? 0u : (uint8_t)code; }

template <typename T>
void swap_buf(DevBuf<T> &a, DevBuf<T> &b) {
    std::swap(a.p, b.p);
    std::swap(a.n, b.n);
}

void invalidate_derived(DScatter &s) {
    s.stream1.valid = s.streamK.valid = false;
    s.stream1.failed = s.streamK.failed = false;
    s.fidx.valid = false;
    s.dcol_valid = false;
    s.sh_valid = false;
    s.slc_w = 0;
    s.cblk.clear();
    s.cblk_cb = 0;
}

// split_rows, n_split and has_split of s from its work items.
void refresh_split(Layer &L, DScatter &s) {
    hipStream_t st = L.stream;
    TmpBuf<uint32_t> flag(L, SILI_TMPKEY(flag)), pos(L, SILI_TMPKEY(pos));
    flag.ensure((size_t)s.rows + 1);
    pos.ensure((size_t)s.rows + 1);
    launch(k_fill0_u32, dim3(nblk(s.rows + 1)), dim3(TPB), 0, st, flag.p, s.rows + 1);
    if (s.nseg > 0) launch(k_split_from_segs, dim3(nblk(s.nseg)), dim3(TPB), 0, st, (const SegDesc *)s.seg.p, s.nseg, flag.p);
    SILI_HIP(hipGetLastError());
    device_exclusive_scan_u32(L, flag.p, pos.p, s.rows + 1);
    uint32_t ns = 0;
    SILI_HIP(hipMemcpyAsync(&ns, pos.p + s.rows, 4, hipMemcpyDeviceToHost, st));
    SILI_HIP(hipStreamSynchronize(st));
    s.n_split = ns;
    s.has_split = ns > 0;
    prepare_split_combine(L, s);
    if (ns > 0) {
        s.split_rows.ensure((size_t)ns + 1);
        launch(k_list_rows, dim3(nblk(s.rows)), dim3(TPB), 0, st, (const uint32_t *)flag.p, (const uint32_t *)pos.p,
               s.rows, s.split_rows.p);
        SILI_HIP(hipGetLastError());
    }
}

// has_split of a block4 orientation from its work items.
void refresh_split_b4(Layer &L, DBlock4 &b) {
    hipStream_t st = L.stream;
    TmpBuf<uint32_t> flag(L, SILI_TMPKEY(flag)), pos(L, SILI_TMPKEY(pos));
    flag.ensure((size_t)b.brows + 1);
    pos.ensure((size_t)b.brows + 1);
    launch(k_fill0_u32, dim3(nblk(b.brows + 1)), dim3(TPB), 0, st, flag.p, b.brows + 1);
    if (b.nseg > 0) launch(k_split_from_segs, dim3(nblk(b.nseg)), dim3(TPB), 0, st, (const SegDesc *)b.seg.p, b.nseg, flag.p);
    SILI_HIP(hipGetLastError());
    device_exclusive_scan_u32(L, flag.p, pos.p, b.brows + 1);
    uint32_t ns = 0;
    SILI_HIP(hipMemcpyAsync(&ns, pos.p + b.brows, 4, hipMemcpyDeviceToHost, st));
    SILI_HIP(hipStreamSynchronize(st));
    b.has_split = ns > 0;
}

StoreArrays arrays_of(DScatter &s, ScatSpare &sp, DevBuf<uint32_t> *perm, uint32_t seg_bytes) {
    StoreArrays A{};
    A.bstart = &s.byte_start;
    A.estart = &s.elem_start;
    A.idx = &s.idx;
    A.elems = &s.val;
    A.flags = nullptr;
    A.perm = perm;
    A.seg = &s.seg;
    A.sp_bstart = &sp.byte_start;
    A.sp_estart = &sp.elem_start;
    A.sp_idx = &sp.idx;
    A.sp_elems = &sp.val;
    A.sp_flags = nullptr;
    A.sp_perm = &sp.perm;
    A.sp_seg = &sp.seg;
    A.rows = s.rows;
    A.nbytes = s.nbytes;
    A.nelems = s.nnz;
    A.nseg = s.nseg;
    A.elem_bytes = 1;
    A.seg_bytes = seg_bytes;
    A.emit_empty = true;
    return A;
}
StoreArrays arrays_of(DBlock4 &b, B4Spare &sp, bool flags, DevBuf<uint32_t> *perm, uint32_t seg_bytes) {
    StoreArrays A{};
    A.bstart = &b.byte_start;
    A.estart = &b.tile_start;
    A.idx = &b.idx;
    A.elems = &b.tiles;
    A.flags = flags ? &b.sparse : nullptr;
    A.perm = perm;
    A.seg = &b.seg;
    A.sp_bstart = &sp.byte_start;
    A.sp_estart = &sp.tile_start;
    A.sp_idx = &sp.idx;
    A.sp_elems = &sp.tiles;
    A.sp_flags = &sp.sparse;
    A.sp_perm = &sp.perm;
    A.sp_seg = &sp.seg;
    A.rows = b.brows;
    A.nbytes = b.nbytes;
    A.nelems = b.ntiles;
    A.nseg = b.nseg;
    A.elem_bytes = 16;
    A.seg_bytes = seg_bytes;
    A.emit_empty = false;
    return A;
}

void swap_store(DScatter &s, ScatSpare &sp, DevBuf<uint32_t> *perm) {
    swap_buf(s.byte_start, sp.byte_start);
    swap_buf(s.elem_start, sp.elem_start);
    swap_buf(s.idx, sp.idx);
    swap_buf(s.val, sp.val);
    swap_buf(s.seg, sp.seg);
    if (perm) swap_buf(*perm, sp.perm);
}
void swap_store(DBlock4 &b, B4Spare &sp, bool flags, DevBuf<uint32_t> *perm) {
    swap_buf(b.byte_start, sp.byte_start);
    swap_buf(b.tile_start, sp.tile_start);
    swap_buf(b.idx, sp.idx);
    swap_buf(b.tiles, sp.tiles);
    swap_buf(b.seg, sp.seg);
    if (flags) swap_buf(b.sparse, sp.sparse);
    if (perm) swap_buf(*perm, sp.perm);
}

// Upper bound of the work items a store will hold after a patch (the seg
// second buffer is sized before any piece points into it).
int64_t seg_bound(int64_t nseg, const std::vector<StagedRow> &old, const std::vector<NewRow> &nu, uint32_t seg_bytes) {
    int64_t n = nseg;
    const uint32_t W = seg_bytes - 4u;
    for (size_t j = 0; j < nu.size(); ++j) {
        n -= old[j].shi - old[j].slo;
        n += (int64_t)(nu[j].cols.size() * 5) / W + 2;  // >= the row's items (5 bytes per varint at most)
    }
    return n;
}

// Upload the patch content and pieces, check every piece against the
// arrays it reads and the second buffers it writes, and launch the splice.
void launch_patch(Layer &L, PatchBuilder &P, std::initializer_list<StoreArrays *> stores,
                  std::initializer_list<uint64_t> remaps) {
    hipStream_t st = L.stream;
    const size_t pieces_off = (P.blob.size() + 63) & ~size_t(63);
    const uint32_t np = (uint32_t)P.pieces.size();
    const size_t total = pieces_off + (size_t)np * sizeof(PatchPiece);
    L.patch_blob.ensure(total + 64);
    const uint64_t dblob = reinterpret_cast<uint64_t>(L.patch_blob.p);
    // remaps' map fields become device addresses
    for (uint64_t ro : remaps) {
        if (ro == ~0ull) continue;
        Remap R;
        std::memcpy(&R, P.blob.data() + ro, sizeof(R));
        R.map += dblob;
        std::memcpy(P.blob.data() + ro, &R, sizeof(R));
    }
    L.pin_patch.ensure(total);
    std::memcpy(L.pin_patch.h, P.blob.data(), P.blob.size());
    PatchPiece *pp = reinterpret_cast<PatchPiece *>(L.pin_patch.h + pieces_off);
    // every piece reads inside one array (or the content) and writes inside
    // one second buffer: checked here, before anything is launched
    std::vector<std::pair<uint64_t, uint64_t>> srcs, dsts;  // [begin, end) bytes
    auto add = [](std::vector<std::pair<uint64_t, uint64_t>> &v, const void *p, size_t bytes) {
        if (p) v.push_back({reinterpret_cast<uint64_t>(p), reinterpret_cast<uint64_t>(p) + bytes});
    };
    for (StoreArrays *A : stores) {
        add(srcs, A->bstart->p, A->bstart->n * 4);
        add(srcs, A->estart->p, A->estart->n * 4);
        add(srcs, A->idx->p, A->idx->n);
        add(srcs, A->elems->p, A->elems->n);
        add(srcs, A->seg->p, A->seg->n * sizeof(SegDesc));
        if (A->flags) add(srcs, A->flags->p, A->flags->n);
        if (A->perm) add(srcs, A->perm->p, A->perm->n * 4);
        add(dsts, A->sp_bstart->p, A->sp_bstart->n * 4);
        add(dsts, A->sp_estart->p, A->sp_estart->n * 4);
        add(dsts, A->sp_idx->p, A->sp_idx->n);
        add(dsts, A->sp_elems->p, A->sp_elems->n);
        add(dsts, A->sp_seg->p, A->sp_seg->n * sizeof(SegDesc));
        if (A->flags) add(dsts, A->sp_flags->p, A->sp_flags->n);
        if (A->perm) add(dsts, A->sp_perm->p, A->sp_perm->n * 4);
    }
    auto inside = [](const std::vector<std::pair<uint64_t, uint64_t>> &v, uint64_t a, uint64_t b) {
        for (const auto &r : v)
            if (a >= r.first && b <= r.second) return true;
        return false;
    };
    for (uint32_t i = 0; i < np; ++i) {
        const PatchPiece &p = P.pieces[i].p;
        const uint64_t es = p.mode == PM_BYTES ? 1 : p.mode == PM_SEG ? sizeof(SegDesc) : 4;
        const bool src_ok = P.pieces[i].src_blob ? p.src + p.n * es <= P.blob.size()
                                                 : inside(srcs, p.src, p.src + p.n * es);
        const bool aux_ok = p.mode != PM_U32_REMAP || (P.pieces[i].aux_blob && p.aux + sizeof(Remap) <= P.blob.size());
        if (!src_ok || !aux_ok || !inside(dsts, p.dst, p.dst + p.n * es))
            throw_error(SILI_ERR_RUNTIME, "row patch: a piece falls outside its arrays (internal error)");
    }
    uint32_t chunks = 0;
    for (uint32_t i = 0; i < np; ++i) {
        PatchPiece p = P.pieces[i].p;
        if (P.pieces[i].src_blob) p.src += dblob;
        if (P.pieces[i].aux_blob) p.aux += dblob;
        p.chunk0 = chunks;
        chunks += (uint32_t)((p.n + chunk_elems(p.mode) - 1) / chunk_elems(p.mode));
        pp[i] = p;
    }
    SILI_HIP(hipMemcpyAsync(L.patch_blob.p, L.pin_patch.h, total, hipMemcpyHostToDevice, st));
    if (chunks > 0)
        launch(k_patch_apply, dim3(chunks), dim3(TPB), 0, st,
               reinterpret_cast<const PatchPiece *>(L.patch_blob.p + pieces_off), np);
    SILI_HIP(hipGetLastError());
}

__global__ void k_copy_bytes(const uint8_t *__restrict__ src, int64_t n, uint8_t *__restrict__ dst) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i < n) dst[i] = src[i];
}

}  // namespace


bool patch_block_row(Layer &L, const BlockRowState &old, const BlockRowState &nu,
                     const std::vector<StagedRow> &w_rows, const StagedRow *b4_row) {
    const uint32_t br = old.br;
    const int64_t r0 = (int64_t)br * 4;
    const uint32_t nr = (uint32_t)std::min<int64_t>(4, L.n_in - r0);
    if (w_rows.size() != nr) return false;
    const bool has_b4 = b4_row != nullptr;
    if (!has_b4 && !nu.tiles.empty()) return false;
    const bool keep_wperm = L.keep_perm && L.Wt_perm.p != nullptr && L.W.nnz > 0;
    const bool keep_bperm = has_b4 && L.B4t_perm.p != nullptr;
    // ---- canonical scattered rows ------------------------------------------------
    std::vector<StagedRow> w_old;
    std::vector<NewRow> w_new;
    // new canonical entry index of each (row, col) of the block row: old
    // start of the row shifted by the edited rows before it, plus its position
    std::vector<int64_t> row_shift(nr, 0);
    {
        int64_t de = 0;
        for (uint32_t li = 0; li < nr; ++li) {
            row_shift[li] = de;
            if (old.rows[li] != nu.rows[li]) {
                NewRow R;
                R.row = (uint32_t)(r0 + li);
                for (const auto &e : nu.rows[li]) {
                    R.cols.push_back(e.first);
                    R.elems.push_back(e.second);
                }
                w_new.push_back(std::move(R));
                w_old.push_back(w_rows[li]);
                de += (int64_t)nu.rows[li].size() - (int64_t)old.rows[li].size();
            }
        }
    }
    auto new_w_index = [&](uint32_t li, uint32_t col) -> uint32_t {
        const auto &v = nu.rows[li];
        const auto it = std::lower_bound(v.begin(), v.end(), std::make_pair(col, (uint8_t)0),
                                         [](const std::pair<uint32_t, uint8_t> &a, const std::pair<uint32_t, uint8_t> &b) {
                                             return a.first < b.first;
                                         });
        return (uint32_t)(w_rows[li].e0 + row_shift[li] + (it - v.begin()));
    };
    // ---- shadow scattered rows: the columns whose (row, byte) sets differ ----------
    std::map<uint32_t, std::vector<std::pair<uint32_t, int>>> t_edit;  // col -> (row, byte + 1 add | -1 remove)
    for (uint32_t li = 0; li < nr; ++li) {
        if (old.rows[li] == nu.rows[li]) continue;
        const uint32_t r = (uint32_t)(r0 + li);
        const auto &a = old.rows[li], &b = nu.rows[li];
        size_t i = 0, k = 0;
        while (i < a.size() || k < b.size()) {
            if (k == b.size() || (i < a.size() && a[i].first < b[k].first)) {
                t_edit[a[i++].first].push_back({r, -1});
            } else if (i == a.size() || b[k].first < a[i].first) {
                t_edit[b[k].first].push_back({r, (int)b[k].second + 1});
                ++k;
            } else {
                if (a[i].second != b[k].second) {
                    t_edit[a[i].first].push_back({r, -1});
                    t_edit[a[i].first].push_back({r, (int)b[k].second + 1});
                }
                ++i;
                ++k;
            }
        }
    }
    // ---- block4: the block row and the block columns whose tiles differ ------------
    const bool b4_changed = has_b4 && old.tiles != nu.tiles;
    std::set<uint32_t> bt_cols;
    if (b4_changed) {
        for (const auto &t : old.tiles) {
            auto it = nu.tiles.find(t.first);
            if (it == nu.tiles.end() || it->second.b != t.second.b) bt_cols.insert(t.first);
        }
        for (const auto &t : nu.tiles)
            if (!old.tiles.count(t.first)) bt_cols.insert(t.first);
    }
    if (w_new.empty() && !b4_changed) return true;  // nothing stored changed
    if (t_edit.size() > STAGE_MAX_ROWS || bt_cols.size() > STAGE_MAX_ROWS) return false;

    // ---- stage the shadow rows -----------------------------------------------------
    StageReq qt, qbt;
    qt.s = &L.Wt;
    qt.perm = keep_wperm ? L.Wt_perm.p : nullptr;
    for (const auto &e : t_edit) qt.rows.push_back(e.first);
    qbt.b = &L.B4t;
    qbt.perm = keep_bperm ? L.B4t_perm.p : nullptr;
    for (uint32_t bc : bt_cols) qbt.rows.push_back(bc);
    {
        std::vector<StageReq *> reqs;
        if (!qt.rows.empty()) reqs.push_back(&qt);
        if (!qbt.rows.empty()) reqs.push_back(&qbt);
        if (!reqs.empty()) stage_rows(L, reqs);
    }

    PatchBuilder P;
    // ---- W remap (Wt_perm values): canonical entries of the edited span ------------
    uint64_t w_remap = ~0ull;
    int64_t w_de_total = 0;
    for (uint32_t li = 0; li < nr; ++li) w_de_total += (int64_t)nu.rows[li].size() - (int64_t)old.rows[li].size();
    if (keep_wperm && !w_new.empty()) {
        const uint32_t E0 = w_old.front().e0, E1 = w_old.back().e1;
        std::vector<uint32_t> map(E1 - E0, 0u);
        for (uint32_t li = 0; li < nr; ++li) {
            const StagedRow &S = w_rows[li];
            if (S.e1 <= E0 || S.e0 >= E1) continue;
            for (uint32_t k = 0; k < S.e1 - S.e0; ++k) {
                const uint32_t col = old.rows[li][k].first;
                const auto &v = nu.rows[li];
                const bool kept = std::binary_search(v.begin(), v.end(), std::make_pair(col, (uint8_t)0),
                                                     [](const std::pair<uint32_t, uint8_t> &a, const std::pair<uint32_t, uint8_t> &b) {
                                                         return a.first < b.first;
                                                     });
                map[S.e0 + k - E0] = kept ? new_w_index(li, col) : 0u;
            }
        }
        Remap R{E0, E1, w_de_total, 0};
        const size_t map_off = P.put(map.data(), map.size() * 4);
        R.map = map_off;  // blob offset; made a device address below
        w_remap = P.put(&R, sizeof(R));
    }
    // ---- B4 remap (B4t_perm values): the block row's tiles ------------------------
    uint64_t b_remap = ~0ull;
    if (keep_bperm && b4_changed) {
        const uint32_t T0 = b4_row->e0, T1 = b4_row->e1;
        std::vector<uint32_t> map(T1 - T0, 0u);
        uint32_t k = 0;
        for (const auto &t : old.tiles) {
            auto it = nu.tiles.find(t.first);
            map[k++] = it == nu.tiles.end() ? 0u : T0 + (uint32_t)std::distance(nu.tiles.begin(), it);
        }
        Remap R{T0, T1, (int64_t)nu.tiles.size() - (int64_t)old.tiles.size(), 0};
        const size_t map_off = P.put(map.data(), map.size() * 4);
        R.map = map_off;
        b_remap = P.put(&R, sizeof(R));
    }

    // ---- new shadow rows --------------------------------------------------------------
    std::vector<NewRow> t_new;
    for (size_t j = 0; j < qt.rows.size(); ++j) {
        const StagedRow &S = qt.out[j];
        const uint32_t c = S.row;
        const auto cols = staged_cols(S);
        const auto &ed = t_edit[c];  // by row, ascending; a row's removal before its add
        NewRow R;
        R.row = c;
        const uint32_t E0 = w_new.empty() ? 0u : w_old.front().e0;
        auto emit = [&](uint32_t r, uint8_t byte, uint32_t old_perm, bool is_new) {
            R.cols.push_back(r);
            R.elems.push_back(byte);
            if (!keep_wperm) return;
            uint32_t v;
            if (r >= r0 && r < r0 + nr) v = new_w_index(r - (uint32_t)r0, c);
            else if (is_new || w_new.empty() || old_perm < E0) v = old_perm;
            else v = (uint32_t)((int64_t)old_perm + w_de_total);
            R.perm.push_back(v);
        };
        size_t i = 0, e = 0;
        while (i < cols.size() || e < ed.size()) {
            if (e < ed.size() && (i == cols.size() || ed[e].first <= cols[i])) {
                const uint32_t r = ed[e].first;
                bool have = i < cols.size() && cols[i] == r;
                uint8_t byte = have ? S.elems[i] : 0;
                const uint32_t op = have && keep_wperm ? S.perm[i] : 0u;
                if (have) ++i;
                bool added = false;
                for (; e < ed.size() && ed[e].first == r; ++e) {
                    if (ed[e].second < 0) {
                        have = false;
                    } else {
                        have = true;
                        added = true;
                        byte = (uint8_t)(ed[e].second - 1);
                    }
                }
                if (have) emit(r, byte, op, added);
            } else {
                emit(cols[i], S.elems[i], keep_wperm ? S.perm[i] : 0u, false);
                ++i;
            }
        }
        t_new.push_back(std::move(R));
    }
    // ---- the new canonical block row and shadow block rows -----------------------------
    std::vector<NewRow> b_new, bt_new;
    std::vector<StagedRow> b_old;
    if (b4_changed) {
        NewRow R;
        R.row = br;
        for (const auto &t : nu.tiles) {
            R.cols.push_back(t.first);
            R.elems.insert(R.elems.end(), t.second.b.begin(), t.second.b.end());
            R.flags.push_back(t.second.sparse);
        }
        b_new.push_back(std::move(R));
        b_old.push_back(*b4_row);
        const uint32_t T0 = b4_row->e0;
        const int64_t dt = (int64_t)nu.tiles.size() - (int64_t)old.tiles.size();
        for (size_t j = 0; j < qbt.rows.size(); ++j) {
            const StagedRow &S = qbt.out[j];
            const uint32_t bc = S.row;
            const auto brs = staged_cols(S);
            std::map<uint32_t, std::pair<std::array<uint8_t, 16>, uint32_t>> ent;
            for (size_t k = 0; k < brs.size(); ++k) {
                std::array<uint8_t, 16> tb;
                std::copy(S.elems.begin() + k * 16, S.elems.begin() + k * 16 + 16, tb.begin());
                ent[brs[k]] = {tb, keep_bperm ? S.perm[k] : 0u};
            }
            ent.erase(br);
            auto it = nu.tiles.find(bc);
            if (it != nu.tiles.end()) {
                std::array<uint8_t, 16> tb;
                for (int li = 0; li < 4; ++li)
                    for (int lj = 0; lj < 4; ++lj) tb[li * 4 + lj] = it->second.b[lj * 4 + li];
                ent[br] = {tb, T0 + (uint32_t)std::distance(nu.tiles.begin(), it)};
            }
            NewRow Rt;
            Rt.row = bc;
            for (const auto &e : ent) {
                Rt.cols.push_back(e.first);
                Rt.elems.insert(Rt.elems.end(), e.second.first.begin(), e.second.first.end());
                if (keep_bperm) {
                    const uint32_t o = e.second.second;
                    Rt.perm.push_back(e.first == br ? o : (o < T0 ? o : (uint32_t)((int64_t)o + dt)));
                }
            }
            bt_new.push_back(std::move(Rt));
        }
    }
    // ---- pieces -------------------------------------------------------------------------
    StoreArrays AW = arrays_of(L.W, L.sp_W, nullptr, L.seg_len);
    StoreArrays AT = arrays_of(L.Wt, L.sp_Wt, keep_wperm ? &L.Wt_perm : nullptr, L.seg_len);
    StoreArrays AB = arrays_of(L.B4, L.sp_B4, true, nullptr, L.seg_len_b4);
    StoreArrays ABt = arrays_of(L.B4t, L.sp_B4t, false, keep_bperm ? &L.B4t_perm : nullptr, L.seg_len_b4);
    // second work-item buffers before any piece points into them
    if (!w_new.empty()) {
        L.sp_W.seg.ensure((size_t)seg_bound(L.W.nseg, w_old, w_new, L.seg_len) + 1);
        L.sp_Wt.seg.ensure((size_t)seg_bound(L.Wt.nseg, qt.out, t_new, L.seg_len) + 1);
    }
    if (b4_changed) {
        L.sp_B4.seg.ensure((size_t)seg_bound(L.B4.nseg, b_old, b_new, L.seg_len_b4) + 1);
        L.sp_B4t.seg.ensure((size_t)seg_bound(L.B4t.nseg, qbt.out, bt_new, L.seg_len_b4) + 1);
    }
    StoreDelta dW, dT, dB, dBt;
    if (!w_new.empty()) {
        dW = plan_store(P, AW, w_old, w_new, ~0ull);
        dT = plan_store(P, AT, qt.out, t_new, w_remap);
    }
    if (b4_changed) {
        dB = plan_store(P, AB, b_old, b_new, ~0ull);
        dBt = plan_store(P, ABt, qbt.out, bt_new, b_remap);
    }
    // ---- upload and launch ----------------------------------------------------------------
    launch_patch(L, P, {&AW, &AT, &AB, &ABt}, {w_remap, b_remap});
    // No wait here: the next host write of the pinned content or the edit
    // lists follows the next staging sync, and later work on the layer is
    // stream-ordered behind the patch.
    // ---- swap and bookkeeping ---------------------------------------------------------------
    if (!w_new.empty()) {
        swap_store(L.W, L.sp_W, nullptr);
        swap_store(L.Wt, L.sp_Wt, keep_wperm ? &L.Wt_perm : nullptr);
        L.W.nbytes += dW.dbytes;
        L.W.nnz += dW.delems;
        L.W.nseg += dW.dseg;
        L.W.n_empty_rows += dW.dempty;
        L.Wt.nbytes += dT.dbytes;
        L.Wt.nnz += dT.delems;
        L.Wt.nseg += dT.dseg;
        L.Wt.n_empty_rows += dT.dempty;
        invalidate_derived(L.W);
        invalidate_derived(L.Wt);
        if (dW.split_maybe_changed) refresh_split(L, L.W);
        if (dT.split_maybe_changed) refresh_split(L, L.Wt);
        if (L.keep_perm && !keep_wperm) L.Wt_perm.reset();  // rebuilt with the shadow on the next update
    }
    if (b4_changed) {
        swap_store(L.B4, L.sp_B4, true, nullptr);
        swap_store(L.B4t, L.sp_B4t, false, keep_bperm ? &L.B4t_perm : nullptr);
        L.B4.nbytes += dB.dbytes;
        L.B4.ntiles += dB.delems;
        L.B4.nseg += dB.dseg;
        L.B4t.nbytes += dBt.dbytes;
        L.B4t.ntiles += dBt.delems;
        L.B4t.nseg += dBt.dseg;
        L.B4.cblk.clear();
        L.B4.cblk_cbb = 0;
        L.B4t.cblk.clear();
        L.B4t.cblk_cbb = 0;
        L.B4.rng_k = L.B4t.rng_k = 0;
        if (dB.split_maybe_changed) refresh_split_b4(L, L.B4);
        if (dBt.split_maybe_changed) refresh_split_b4(L, L.B4t);
    }
    // a removed or requantized weight may have been the last code 8
    if (L.has_nonfinite) refresh_nonfinite(L);
    return true;
}

void patch_blocks_rebuild_shadows(Layer &L, const std::vector<const PendingBlock *> &blocks) {
    hipStream_t st = L.stream;
    // canonical rows and block rows that changed, in store order
    std::vector<StagedRow> w_old, b_old;
    std::vector<NewRow> w_new, b_new;
    for (const PendingBlock *pb : blocks) {
        const BlockRowState &o = pb->orig.state, &n = pb->cur;
        for (size_t li = 0; li < pb->orig.w.size(); ++li) {
            if (o.rows[li] == n.rows[li]) continue;
            NewRow R;
            R.row = pb->orig.w[li].row;
            for (const auto &e : n.rows[li]) {
                R.cols.push_back(e.first);
                R.elems.push_back(e.second);
            }
            w_old.push_back(pb->orig.w[li]);
            w_new.push_back(std::move(R));
        }
        if (pb->orig.has_b4 && o.tiles != n.tiles) {
            NewRow R;
            R.row = n.br;
            for (const auto &t : n.tiles) {
                R.cols.push_back(t.first);
                R.elems.insert(R.elems.end(), t.second.b.begin(), t.second.b.end());
                R.flags.push_back(t.second.sparse);
            }
            b_old.push_back(pb->orig.b);
            b_new.push_back(std::move(R));
        } else if (!pb->orig.has_b4 && !n.tiles.empty()) {
            throw_error(SILI_ERR_RUNTIME, "policy flush: tiles on a layer without a block4 store (internal error)");
        }
    }
    if (w_new.empty() && b_new.empty()) return;
    PatchBuilder P;
    StoreArrays AW = arrays_of(L.W, L.sp_W, nullptr, L.seg_len);
    StoreArrays AB = arrays_of(L.B4, L.sp_B4, true, nullptr, L.seg_len_b4);
    StoreDelta dW, dB;
    if (!w_new.empty()) {
        L.sp_W.seg.ensure((size_t)seg_bound(L.W.nseg, w_old, w_new, L.seg_len) + 1);
        dW = plan_store(P, AW, w_old, w_new, ~0ull);
    }
    if (!b_new.empty()) {
        L.sp_B4.seg.ensure((size_t)seg_bound(L.B4.nseg, b_old, b_new, L.seg_len_b4) + 1);
        dB = plan_store(P, AB, b_old, b_new, ~0ull);
    }
    launch_patch(L, P, {&AW, &AB}, {});
    if (!w_new.empty()) {
        swap_store(L.W, L.sp_W, nullptr);
        L.W.nbytes += dW.dbytes;
        L.W.nnz += dW.delems;
        L.W.nseg += dW.dseg;
        L.W.n_empty_rows += dW.dempty;
        invalidate_derived(L.W);
        if (dW.split_maybe_changed) refresh_split(L, L.W);
        // the shadow (and its permutation, when kept) from the canonical store
        DevBuf<uint32_t> rows, cols;
        rows.ensure((size_t)L.W.nnz + 1);
        cols.ensure((size_t)L.W.nnz + 1);
        if (L.W.nnz > 0) decode_scattered(L, rows.p, cols.p);
        build_shadow(L, L.W, rows.p, cols.p, L.Wt);
    }
    if (!b_new.empty()) {
        swap_store(L.B4, L.sp_B4, true, nullptr);
        L.B4.rng_k = 0;
        L.B4.nbytes += dB.dbytes;
        L.B4.ntiles += dB.delems;
        L.B4.nseg += dB.dseg;
        if (dB.split_maybe_changed) refresh_split_b4(L, L.B4);
        // both block4 orientations (and the shadow's permutation) rebuilt
        // from the patched canonical tiles, their flags carried along
        const int64_t T = L.B4.ntiles;
        DevBuf<uint32_t> br, bc;
        DevBuf<uint8_t> tiles, flags;
        br.ensure((size_t)T + 1);
        bc.ensure((size_t)T + 1);
        tiles.ensure((size_t)T * 16 + 16);
        flags.ensure((size_t)T + 1);
        if (T > 0) {
            launch_decode_b4(L.B4.plan(), br.p, bc.p, st);
            launch(k_copy_bytes, dim3(nblk(T * 16)), dim3(TPB), 0, st, (const uint8_t *)L.B4.tiles.p, T * 16, tiles.p);
            launch(k_copy_bytes, dim3(nblk(T)), dim3(TPB), 0, st, (const uint8_t *)L.B4.sparse.p, T, flags.p);
            SILI_HIP(hipGetLastError());
        }
        build_block4(L, T, br.p, bc.p, tiles.p, flags.p);
    }
    if (L.has_nonfinite) refresh_nonfinite(L);
    SILI_HIP(hipStreamSynchronize(st));
}

}  // namespace sili
