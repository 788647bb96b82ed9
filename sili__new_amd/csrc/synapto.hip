// synapto.hip -- the bulk synaptogenesis step on the GPU: magnitude prune,
// regrowth at host-supplied candidates, block4 demote / promote, and the
// rebuild of both stores, all by device sort, scan and compaction.
//
// Selection policy (new; the reference prunes by importance, row by row,
// delta_csr_memory.hpp:1019-1258): the k = llround(prune_frac * N) stored
// synapses (scattered + live block4 slots) with the smallest
// |fl32(dec(code) * S(r,c))| (fp32 bit order, so NaN sorts above inf) are
// removed, ties by (row, col) ascending; as many are regrown at the first
// valid candidates in list order.  Structural rules follow the reference:
//   - a pruned block4 slot is zeroed; a touched tile whose live count
//     (nonzero bytes) drops below 2 is demoted, its remaining slot becoming
//     a scattered synapse with both nibbles requantized (code 8 -> 0) and
//     swapped into the scattered byte order (delta_csr_memory.hpp:949-999,
//     1203-1225);
//   - an insert whose 4x4 window holds a (surviving) tile writes that tile's
//     slot (delta_csr_memory.hpp:620-646); otherwise it is a scattered
//     insert, and every window that received one and then holds >= 2
//     scattered synapses is promoted into a new tile (:648-700).
// Phase order: select -> prune -> demote -> insert -> promote -> rebuild.
//
// Keys: a synapse is (row, col) packed as rc = row << 32 | col (rows and
// cols < 2^31, so real keys never reach KEY_NONE); sorted rc arrays serve
// the membership tests by binary search.
#include "sili_hip.h"
#include "layer.hpp"
#include "wave.hpp"

#include <cmath>
#include <vector>

namespace sili {

namespace {

constexpr unsigned TPB = 256;
inline unsigned nblk(int64_t n) { return (unsigned)((n + TPB - 1) / TPB); }
constexpr uint64_t KEY_NONE = ~0ull;

__device__ __forceinline__ uint64_t rc_key(uint32_t r, uint32_t c) { return ((uint64_t)r << 32) | c; }
__device__ __forceinline__ uint32_t requant(uint32_t code) { return code == 8u ? 0u : code; }

// First index in sorted a[0, n) with a[i] >= key.
__device__ __forceinline__ int64_t lower_bound_u64(const uint64_t *a, int64_t n, uint64_t key) {
    int64_t lo = 0, hi = n;
    while (lo < hi) {
        const int64_t mid = (lo + hi) >> 1;
        if (a[mid] < key) lo = mid + 1;
        else hi = mid;
    }
    return lo;
}
__device__ __forceinline__ bool contains_u64(const uint64_t *a, int64_t n, uint64_t key) {
    const int64_t i = lower_bound_u64(a, n, key);
    return i < n && a[i] == key;
}
// Surviving tile of window (br, bc), or -1.  tkey: canonical tile keys
// br*bcols + bc, ascending (the store's own order).
__device__ __forceinline__ int64_t find_tile(const uint64_t *tkey, int64_t T, const uint8_t *alive,
                                             uint64_t wkey) {
    const int64_t t = lower_bound_u64(tkey, T, wkey);
    return (t < T && tkey[t] == wkey && alive[t]) ? t : -1;
}

__global__ void k_fill_u8(uint8_t *p, int64_t n, uint8_t v) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i < n) p[i] = v;
}
__global__ void k_fill_u32(uint32_t *p, int64_t n, uint32_t v) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i < n) p[i] = v;
}
__global__ void k_iota32(uint32_t *p, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i < n) p[i] = (uint32_t)i;
}

// Keys of every stored synapse: scattered entries [0, Ns), then the 16
// slots of every tile [Ns, Ns + 16T) (dead or out-of-range slots get
// KEY_NONE / 0xFFFFFFFF so they sort after every live synapse).
__global__ void k_syn_keys(int64_t Ns, const uint32_t *srow, const uint32_t *scol, const uint8_t *sval,
                           int64_t T, const uint32_t *tbr, const uint32_t *tbc, const uint8_t *tiles,
                           int64_t n_in, int64_t n_out, ScaleView sc, uint64_t *rc, uint32_t *absw) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i < Ns) {
        const uint32_t r = srow[i], c = scol[i];
        const float w = fp4_decode((uint32_t)sval[i] >> 4) * scale_at(sc, r, c);
        rc[i] = rc_key(r, c);
        absw[i] = __builtin_bit_cast(uint32_t, w) & 0x7FFFFFFFu;
    } else if (i - Ns < 16 * T) {
        const int64_t s = i - Ns;
        const int64_t t = s >> 4;
        const uint32_t sl = (uint32_t)(s & 15), lj = sl >> 2, li = sl & 3u;
        const uint32_t r = tbr[t] * 4u + li, c = tbc[t] * 4u + lj;
        const uint32_t b = tiles[s];
        if (b == 0u || r >= n_in || c >= n_out) {
            rc[i] = KEY_NONE;
            absw[i] = 0xFFFFFFFFu;
        } else {
            const float w = fp4_decode(b & 0xFu) * scale_at(sc, r, c);
            rc[i] = rc_key(r, c);
            absw[i] = __builtin_bit_cast(uint32_t, w) & 0x7FFFFFFFu;
        }
    }
}

// ---- radix select of the k smallest (|w| bits, row, col) ------------------
// Histogram levels of at most 12 bits, from the top, over the 31 |w| bits of
// the live slots fix the k-th smallest value t and how many live slots lie
// below it; every slot below t is pruned.  Of the slots equal to t, the
// first ones in (row, col) order are taken by a second select over their
// (row << 32 | col) keys (unique).  The same set as a full sort by
// (|w|, row, col) gives, without sorting every slot.
struct SelState {
    unsigned long long prefix;  // the high bits of the threshold fixed so far
    unsigned long long need;    // keys still to take at or above the prefix
    unsigned long long less;    // keys below the prefix
    unsigned long long pad;     // keys in the chosen bin (after the last level: the ties)
};

// A selection's initial state, written by a kernel (a host copy of a stack
// value costs a runtime staging launch).
__global__ void k_put_state(SelState *p, SelState v) { *p = v; }

// Histogram of bits [shift, shift + width) of the keys below `limit` whose
// bits above shift + width equal the state's prefix (level > 0).  Lanes of a
// wave that share a bin add once (ties concentrate on one bin).
template <typename K>
__global__ void k_sel_hist(const K *__restrict__ keys, int64_t n, K limit, int shift, int width, int level,
                           const SelState *__restrict__ st, uint32_t *__restrict__ hist) {
    __shared__ uint32_t s_h[4096];
    for (uint32_t b = threadIdx.x; b < 4096u; b += TPB) s_h[b] = 0u;
    __syncthreads();
    const unsigned long long prefix = level > 0 ? st->prefix : 0ull;
    const uint32_t mask = (1u << width) - 1u, lane = threadIdx.x & 63u;
    const int64_t stride = (int64_t)gridDim.x * TPB;
    // every lane runs the same trip count (the wave-level ballots below)
    const int64_t trips = (n + stride - 1) / stride;
    for (int64_t j = 0; j < trips; ++j) {
        const int64_t i = j * stride + (int64_t)blockIdx.x * TPB + threadIdx.x;
        bool act = false;
        uint32_t bin = 0;
        if (i < n) {
            const K v = keys[i];
            if (v < limit && (level == 0 || ((unsigned long long)v >> (shift + width)) == prefix)) {
                act = true;
                bin = (uint32_t)((unsigned long long)v >> shift) & mask;
            }
        }
        const uint64_t am = __ballot(act);
        if (!am) continue;
        const uint32_t leader = (uint32_t)__builtin_ctzll(am);
        const uint32_t b0 = (uint32_t)__shfl((int)bin, (int)leader, 64);
        const uint64_t same = __ballot(act && bin == b0);
        if (same == am) {
            if (lane == leader) atomicAdd(&s_h[b0], (uint32_t)__popcll(am));
        } else if (act) {
            atomicAdd(&s_h[bin], 1u);
        }
    }
    __syncthreads();
    for (uint32_t b = threadIdx.x; b < 4096u; b += TPB)
        if (s_h[b]) atomicAdd(hist + b, s_h[b]);
}

// One block: the bin holding the need-th key; the state moves to it.
__global__ __launch_bounds__(TPB) void k_sel_find(const uint32_t *__restrict__ hist, uint32_t nbins, int width,
                                                  SelState *__restrict__ st) {
    __shared__ unsigned long long s_part[TPB / 64];
    const uint32_t t = threadIdx.x, per = (nbins + TPB - 1) / TPB;
    unsigned long long mine = 0;
    for (uint32_t j = 0; j < per; ++j) {
        const uint32_t b = t * per + j;
        mine += b < nbins ? hist[b] : 0u;
    }
    unsigned long long incl = mine;
    for (int off = 1; off < 64; off <<= 1) {
        const unsigned long long y = __shfl_up(incl, off, 64);
        if ((t & 63u) >= (uint32_t)off) incl += y;
    }
    if ((t & 63u) == 63u) s_part[t >> 6] = incl;
    __syncthreads();
    unsigned long long before = incl - mine;
    for (uint32_t w = 0; w < (t >> 6); ++w) before += s_part[w];
    const unsigned long long need = st->need;
    __syncthreads();
    if (before < need && need <= before + mine) {
        unsigned long long c = before;
        for (uint32_t j = 0; j < per; ++j) {
            const uint32_t b = t * per + j;
            const uint32_t h = b < nbins ? hist[b] : 0u;
            if (c + h >= need) {
                st->prefix = (st->prefix << width) | b;
                st->need = need - c;
                st->less += c;
                st->pad = h;  // at the last level: the keys equal to the threshold
                break;
            }
            c += h;
        }
    }
}

// Per slot: (below t) in the low word, (equal to t) in the high word, for
// one scan that places both; dead slots (0xFFFFFFFF) are neither.
// The selection's compaction in slot order without a scan over the slots:
// k_sel_count writes each block's (below, at) counts packed in one word,
// an exclusive scan over the blocks gives their offsets, and k_sel_place
// puts each slot below the threshold into order[] and each slot at it into
// the tie list (with its key), ranked within its block by wave ballots.
__device__ __forceinline__ void sel_flags(const uint32_t *absw, int64_t M, uint32_t t, int64_t i, bool &lo, bool &eq) {
    const uint32_t v = i < M ? absw[i] : 0xFFFFFFFFu;
    lo = i < M && v < t;
    eq = i < M && v == t;
}
__global__ void k_sel_count(const uint32_t *__restrict__ absw, int64_t M, const SelState *__restrict__ st,
                            uint64_t *__restrict__ bcnt) {
    __shared__ uint32_t s_lo[TPB / 64], s_eq[TPB / 64];
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;  // every lane reaches the ballots
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    bool lo, eq;
    sel_flags(absw, M, (uint32_t)st->prefix, i, lo, eq);
    const unsigned long long mlo = __ballot(lo), meq = __ballot(eq);
    if (lane == 0) {
        s_lo[wave] = (uint32_t)__popcll(mlo);
        s_eq[wave] = (uint32_t)__popcll(meq);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t a = 0, b = 0;
        for (uint32_t w = 0; w < TPB / 64; ++w) {
            a += s_lo[w];
            b += s_eq[w];
        }
        bcnt[blockIdx.x] = a | (b << 32);
    }
}
__global__ void k_sel_place(const uint32_t *__restrict__ absw, const uint64_t *__restrict__ rc, int64_t M,
                            const SelState *__restrict__ st, const uint64_t *__restrict__ boff,
                            uint32_t *__restrict__ order, uint32_t *__restrict__ tie_idx,
                            uint64_t *__restrict__ tie_key) {
    __shared__ uint32_t s_lo[TPB / 64], s_eq[TPB / 64];
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    bool lo, eq;
    sel_flags(absw, M, (uint32_t)st->prefix, i, lo, eq);
    const unsigned long long mlo = __ballot(lo), meq = __ballot(eq);
    if (lane == 0) {
        s_lo[wave] = (uint32_t)__popcll(mlo);
        s_eq[wave] = (uint32_t)__popcll(meq);
    }
    __syncthreads();
    const uint64_t base = boff[blockIdx.x];
    uint64_t plo = (uint32_t)base, peq = base >> 32;
    for (uint32_t w = 0; w < wave; ++w) {
        plo += s_lo[w];
        peq += s_eq[w];
    }
    const unsigned long long below = (1ull << lane) - 1ull;
    if (lo) order[plo + (uint64_t)__popcll(mlo & below)] = (uint32_t)i;
    if (eq) {
        const uint64_t p = peq + (uint64_t)__popcll(meq & below);
        tie_idx[p] = (uint32_t)i;
        tie_key[p] = rc[i];
    }
}

// Ties whose key is at most the take-th smallest (flags for a scan).
__global__ void k_sel_tie_flags(const uint64_t *__restrict__ tie_key, int64_t n, const SelState *__restrict__ st,
                                uint32_t *__restrict__ flags) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i <= n) flags[i] = (i < n && tie_key[i] <= st->prefix) ? 1u : 0u;
}
__global__ void k_sel_tie_scatter(const uint32_t *__restrict__ flags, const uint32_t *__restrict__ pos,
                                  const uint32_t *__restrict__ tie_idx, int64_t n, uint32_t *__restrict__ order) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i < n && flags[i]) order[pos[i]] = tie_idx[i];
}

// The live slots: the sum of the first histogram level (every live key).
__global__ void k_hist_sum(const uint32_t *__restrict__ hist, uint32_t nbins, unsigned long long *out) {
    __shared__ unsigned long long s_part[TPB / 64];
    unsigned long long v = 0;
    for (uint32_t b = threadIdx.x; b < nbins; b += TPB) v += hist[b];
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    if ((threadIdx.x & 63u) == 0u) s_part[threadIdx.x >> 6] = v;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long t = 0;
        for (uint32_t w = 0; w < TPB / 64; ++w) t += s_part[w];
        *out = t;
    }
}

__global__ void k_copy_u32(const uint32_t *__restrict__ src, int64_t n, uint32_t *__restrict__ dst) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i < n) dst[i] = src[i];
}

// Explicit prune list: the slot of every (row, col) key, looked up in the
// (row, col)-sorted slot keys; a key that is not stored sets *missing.  A
// synapse can be stored twice, in its row and in a tile slot (a tile slot
// an update made live over a scattered synapse): PRUNE_TILE in a key picks
// the tile slot, otherwise the scattered entry (slot indices < Ns).
__global__ void k_find_slots(const uint64_t *keys, int64_t n, const uint64_t *rc_sorted, const uint32_t *perm,
                             int64_t M, int64_t Ns, uint32_t *order, int *missing) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i >= n) return;
    const bool tile = (keys[i] & PRUNE_TILE) != 0;
    const uint64_t key = keys[i] & ~PRUNE_TILE;
    for (int64_t p = lower_bound_u64(rc_sorted, M, key); p < M && rc_sorted[p] == key; ++p)
        if (((int64_t)perm[p] >= Ns) == tile) {
            order[i] = perm[p];
            return;
        }
    order[i] = 0u;
    atomicOr(missing, 1);
}

// Number of live synapses: the KEY_NONE entries sort last.
__global__ void k_count_live(const uint64_t *rc_sorted, int64_t n, unsigned long long *out) {
    if (blockIdx.x == 0 && threadIdx.x == 0) *out = (unsigned long long)lower_bound_u64(rc_sorted, n, KEY_NONE);
}

__global__ void k_gather_u8_by(const uint8_t *src, const uint32_t *perm, int64_t n, uint8_t *dst) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i < n) dst[i] = src[perm[i]];
}

__global__ void k_tile_wkeys(const uint32_t *tbr, const uint32_t *tbc, int64_t T, uint64_t bcols,
                             uint64_t *tkey) {
    const int64_t t = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (t < T) tkey[t] = (uint64_t)tbr[t] * bcols + tbc[t];
}

// The k smallest: order[] lists synapse indices by (|w|, row, col).
__global__ void k_syn_prune(const uint32_t *order, int64_t k, int64_t Ns, uint8_t *s_removed, uint8_t *tbytes,
                            uint8_t *touched) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i >= k) return;
    const uint32_t e = order[i];
    if ((int64_t)e < Ns) {
        s_removed[e] = 1;
    } else {
        const int64_t s = (int64_t)e - Ns;
        tbytes[s] = 0;
        touched[s >> 4] = 1;
    }
}

// Touched tiles with live < 2 die; their in-range live slot (at most one)
// becomes a scattered synapse (dem_key / dem_byte per tile).
__global__ void k_syn_demote(int64_t T, const uint32_t *tbr, const uint32_t *tbc, const uint8_t *tbytes,
                             const uint8_t *touched, int64_t n_in, int64_t n_out, uint8_t *alive,
                             uint64_t *dem_key, uint8_t *dem_byte, unsigned long long *n_demoted) {
    const int64_t t = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (t >= T) return;
    dem_key[t] = KEY_NONE;
    dem_byte[t] = 0;
    alive[t] = 1;
    if (!touched[t]) return;
    int live = 0;
    for (int s = 0; s < 16; ++s) live += tbytes[t * 16 + s] != 0;
    if (live >= 2) return;
    alive[t] = 0;
    atomicAdd(n_demoted, 1ull);
    for (uint32_t s = 0; s < 16u; ++s) {
        const uint32_t b = tbytes[t * 16 + s];
        const uint32_t r = tbr[t] * 4u + (s & 3u), c = tbc[t] * 4u + (s >> 2);
        if (b == 0u || r >= n_in || c >= n_out) continue;
        dem_key[t] = rc_key(r, c);
        dem_byte[t] = (uint8_t)((requant(b & 0xFu) << 4) | requant(b >> 4));
    }
}

// The scattered set after prune + demote, unsorted: [0, Ns) survivors,
// [Ns, Ns + T) demoted slots, [Ns + T, Ns + T + n_cand) scattered inserts
// (filled later); KEY_NONE marks no entry.
__global__ void k_syn_set1(int64_t Ns, int64_t T, const uint64_t *rc, const uint8_t *sval,
                           const uint8_t *s_removed, const uint64_t *dem_key, const uint8_t *dem_byte,
                           uint64_t *key, uint8_t *byte) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i < Ns) {
        key[i] = s_removed[i] ? KEY_NONE : rc[i];
        byte[i] = sval[i];
    } else if (i < Ns + T) {
        key[i] = dem_key[i - Ns];
        byte[i] = dem_byte[i - Ns];
    }
}

// Static validity of each candidate: in range, not just pruned, not stored
// (scattered after prune + demote, or a live slot of a surviving tile).
// Valid ones get their rc key, the rest KEY_NONE.  Read off the stores as
// they were before the step: a position is taken exactly when it held a
// synapse there -- an entry of the scattered store, or a nonzero slot byte of
// a tile -- whether this step pruned it (it may not regrow in the step that
// pruned it), kept it, or moved it from a demoted tile to the scattered set.
// rc_scat: the scattered entries' (row << 32 | col) keys in store order
// (ascending); tiles_old: the tiles' bytes before the step.
__global__ void k_syn_cand_static(int64_t n_cand, const int32_t *cr, const int32_t *cc, int64_t n_in,
                                  int64_t n_out, const uint64_t *rc_scat, int64_t Ns, const uint64_t *tkey,
                                  int64_t T, const uint8_t *tiles_old, uint64_t bcols, uint64_t *ckey) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i >= n_cand) return;
    const int32_t r = cr[i], c = cc[i];
    uint64_t key = KEY_NONE;
    if (r >= 0 && r < n_in && c >= 0 && c < n_out) {
        const uint64_t rc = rc_key((uint32_t)r, (uint32_t)c);
        bool ok = !contains_u64(rc_scat, Ns, rc);
        if (ok) {
            const uint64_t wkey = (uint64_t)(r >> 2) * bcols + (uint64_t)(c >> 2);
            const int64_t t = lower_bound_u64(tkey, T, wkey);
            if (t < T && tkey[t] == wkey && tiles_old[t * 16 + (c & 3) * 4 + (r & 3)] != 0) ok = false;
        }
        if (ok) key = rc;
    }
    ckey[i] = key;
}

// First occurrence (in list order) of each valid candidate position: the
// stable sort keeps equal keys in ascending candidate index.
__global__ void k_syn_first(int64_t n_cand, const uint64_t *ckey_sorted, const uint32_t *cidx_sorted,
                            uint32_t *first) {
    const int64_t p = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (p >= n_cand) return;
    const uint64_t k = ckey_sorted[p];
    if (k == KEY_NONE) return;
    if (p == 0 || ckey_sorted[p - 1] != k) first[cidx_sorted[p]] = 1u;
}

// Apply the accepted candidates (first valid ones, rank < k_target): write
// the slot of a surviving tile, else emit a scattered insert + its window.
__global__ void k_syn_insert(int64_t n_cand, const uint32_t *first, const uint32_t *rank, int64_t k_target,
                             const int32_t *cr, const int32_t *cc, const float *cv, const float *cs,
                             uint32_t default_imp, ScaleView sc, const uint64_t *tkey, int64_t T,
                             const uint8_t *alive, uint8_t *tbytes, uint8_t *tins, uint64_t bcols,
                             uint64_t *ins_key, uint8_t *ins_byte, uint64_t *win, unsigned long long *n_grown) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i >= n_cand) return;
    ins_key[i] = KEY_NONE;
    ins_byte[i] = 0;
    win[i] = KEY_NONE;
    if (!first[i] || (int64_t)rank[i] >= k_target) return;
    atomicAdd(n_grown, 1ull);
    const uint32_t r = (uint32_t)cr[i], c = (uint32_t)cc[i];
    const float S = scale_at(sc, r, c);
    const uint32_t wc = fp4_encode(cv[i] / S);
    const uint32_t ic = cs ? fp4_encode(cs[i]) : (default_imp & 0xFu);
    const uint64_t wkey = (uint64_t)(r >> 2) * bcols + (uint64_t)(c >> 2);
    const int64_t t = find_tile(tkey, T, alive, wkey);
    if (t >= 0) {
        tbytes[t * 16 + (c & 3u) * 4u + (r & 3u)] = (uint8_t)((ic << 4) | wc);
        tins[t] = 1;  // an insert into an existing tile re-encodes it (maybe_compress)
    } else {
        ins_key[i] = rc_key(r, c);
        ins_byte[i] = (uint8_t)((wc << 4) | ic);
        win[i] = wkey;
    }
}

// One thread per distinct touched window: count its scattered synapses
// (final set, sorted); >= 2 makes a new tile (nibbles requantized and
// swapped into the tile byte order) and removes them from the set.
__global__ void k_syn_promote(int64_t n_win, const uint64_t *win_sorted, const uint64_t *key2, int64_t n2,
                              const uint8_t *byte2, uint64_t bcols, int64_t n_in, uint8_t *removed2,
                              uint32_t *nt_flag, uint32_t *nt_br, uint32_t *nt_bc, uint8_t *nt_bytes) {
    const int64_t p = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (p >= n_win) return;
    nt_flag[p] = 0u;
    const uint64_t w = win_sorted[p];
    if (w == KEY_NONE || (p > 0 && win_sorted[p - 1] == w)) return;
    const uint32_t br = (uint32_t)(w / bcols), bc = (uint32_t)(w % bcols);
    int64_t lo[4], hi[4];
    int cnt = 0;
    for (uint32_t li = 0; li < 4u; ++li) {
        const uint32_t r = br * 4u + li;
        if (r >= n_in) { lo[li] = hi[li] = 0; continue; }
        lo[li] = lower_bound_u64(key2, n2, rc_key(r, bc * 4u));
        hi[li] = lower_bound_u64(key2, n2, rc_key(r, bc * 4u + 4u));
        cnt += (int)(hi[li] - lo[li]);
    }
    if (cnt < 2) return;
    uint8_t d[16] = {0};
    for (uint32_t li = 0; li < 4u; ++li)
        for (int64_t e = lo[li]; e < hi[li]; ++e) {
            const uint32_t c = (uint32_t)(key2[e] & 0xFFFFFFFFu);
            const uint32_t b = byte2[e];
            d[(c - bc * 4u) * 4u + li] = (uint8_t)(requant(b >> 4) | (requant(b & 0xFu) << 4));
            removed2[e] = 1;
        }
    nt_flag[p] = 1u;
    nt_br[p] = br;
    nt_bc[p] = bc;
    for (int s = 0; s < 16; ++s) nt_bytes[p * 16 + s] = d[s];
}

__global__ void k_flag_final(int64_t n2, const uint64_t *key2, const uint8_t *removed2, uint32_t *flag) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i < n2) flag[i] = (key2[i] != KEY_NONE && !removed2[i]) ? 1u : 0u;
}

__global__ void k_emit_final(int64_t n2, const uint64_t *key2, const uint8_t *byte2, const uint32_t *flag,
                             const uint32_t *pos, uint32_t *rows, uint32_t *cols, uint8_t *bytes) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i >= n2 || !flag[i]) return;
    const uint32_t o = pos[i];
    rows[o] = (uint32_t)(key2[i] >> 32);
    cols[o] = (uint32_t)(key2[i] & 0xFFFFFFFFu);
    bytes[o] = byte2[i];
}

// ptrs[r] = first index of row r in rows[0, n) (sorted), r in [0, nrows].
__global__ void k_row_ptrs(const uint32_t *rows, int64_t n, int64_t nrows, uint32_t *ptrs) {
    const int64_t r = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (r > nrows) return;
    int64_t lo = 0, hi = n;
    while (lo < hi) {
        const int64_t mid = (lo + hi) >> 1;
        if ((int64_t)rows[mid] < r) lo = mid + 1;
        else hi = mid;
    }
    ptrs[r] = (uint32_t)lo;
}

// Tiles out: surviving old tiles [0, T) then promoted windows [T, T + n_win).
__global__ void k_tile_flags(int64_t T, const uint8_t *alive, int64_t n_win, const uint32_t *nt_flag,
                             uint32_t *flag) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i < T) flag[i] = alive[i] ? 1u : 0u;
    else if (i < T + n_win) flag[i] = nt_flag[i - T];
}

// Output tiles with their encoding (tile_is_sparse): a surviving tile keeps
// its own unless it received an insert; inserted and promoted tiles are
// encoded by their live count (block4.hpp:1193-1205, 1226-1290).
// counter += 1 for each tile i > 0 (other than the second run's first) whose
// canonical key is not above its predecessor's: runs [0, head) and
// [head, n) must each be strictly increasing
__global__ void k_tile_runs_order(const uint32_t *__restrict__ br, const uint32_t *__restrict__ bc, int64_t n,
                                  int64_t head, uint64_t bcols, unsigned long long *__restrict__ bad) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i <= 0 || i >= n || i == head) return;
    const uint64_t a = (uint64_t)br[i - 1] * bcols + bc[i - 1], b = (uint64_t)br[i] * bcols + bc[i];
    if (a >= b) atomicAdd(bad, 1ull);
}

__global__ void k_emit_tiles(int64_t T, const uint32_t *tbr, const uint32_t *tbc, const uint8_t *tbytes,
                             const uint8_t *tsparse, const uint8_t *tins, uint32_t sp, int64_t n_win,
                             const uint32_t *nt_br, const uint32_t *nt_bc, const uint8_t *nt_bytes,
                             const uint32_t *flag, const uint32_t *pos, uint32_t *obr, uint32_t *obc,
                             uint8_t *obytes, uint8_t *osparse) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i >= T + n_win || !flag[i]) return;
    const uint32_t o = pos[i];
    const bool old = i < T;
    const int64_t j = old ? i : i - T;
    obr[o] = old ? tbr[j] : nt_br[j];
    obc[o] = old ? tbc[j] : nt_bc[j];
    const uint8_t *src = old ? tbytes + j * 16 : nt_bytes + j * 16;
    uint32_t live = 0;
    for (int s = 0; s < 16; ++s) {
        obytes[(int64_t)o * 16 + s] = src[s];
        live += src[s] != 0;
    }
    osparse[o] = (old && !tins[j]) ? tsparse[j] : (live <= sp ? 1u : 0u);
}

template <typename T>
T read_back(Layer &L, const T *d) {
    T h{};
    ReadBack rb(L);
    rb.add(&h, d, sizeof(T));
    rb.wait();
    return h;
}

// ---- 64-bit keys in order by (major, minor), with no wait on the host ------
// The step's key sets are (row << 32 | col) pairs or window numbers
// (block row * bcols + block col), with KEY_NONE for empty entries.  Rather
// than a radix sort over all the key bits (two dozen launches for the final
// set), the entries are counted per major, placed in their major's segment
// (one atomic per run of equal majors in a wave), and each segment ordered
// by (minor, entry index): one wave per segment, a bitonic
// network over the lanes (up to 64) or in the wave's LDS (up to KO_CAP), and
// for a longer segment one block on it in global memory.  Equal keys end up in
// ascending entry index, as a stable sort leaves them.  KEY_NONE entries form
// one more segment after every major, left in no particular order (the
// step's readers skip them).  Six launches; nothing is read back.
constexpr uint32_t KO_BINS = 16384 + 1024;
// KO_CAP bounds the LDS network's segment (KO_WAVES * KO_CAP * 8 bytes of LDS
// per block): at 2048 the 64 KiB block left 8 waves per CU, and the launch
// over 16384 short segments took 25 us whatever their lengths.
constexpr uint32_t KO_WAVES = 4, KO_CAP = 512, KO_LONG_LDS = 8192, KO_LONG_MAX_BLOCKS = 65536;

struct KeySplit {
    uint64_t div;    // 0: major = key >> 32, minor = low 32 bits
    uint32_t n_maj;  // majors are < n_maj; KEY_NONE takes major n_maj
    __device__ __forceinline__ uint32_t major(uint64_t k) const {
        if (k == KEY_NONE) return n_maj;
        const uint64_t m = div ? k / div : k >> 32;
        return m < n_maj ? (uint32_t)m : n_maj;  // (never: every real key's major is < n_maj)
    }
    __device__ __forceinline__ uint32_t minor(uint64_t k) const { return div ? (uint32_t)(k % div) : (uint32_t)k; }
    __device__ __forceinline__ uint64_t key(uint32_t m, uint32_t mn) const {
        return div ? (uint64_t)m * div + mn : ((uint64_t)m << 32) | mn;
    }
};

// A wave's runs of equal majors (the final set's survivors arrive sorted, so
// a run is often the whole wave): the run's first lane, its length and this
// lane's rank in it.  Every lane must be active.
struct KoRun {
    uint32_t head, len, rank;
};
__device__ __forceinline__ KoRun ko_run(uint32_t m, uint32_t lane) {
    const uint32_t prev = (uint32_t)__shfl_up((int)m, 1, 64);
    const uint64_t bnd = __ballot(lane == 0u || prev != m);
    const uint64_t upto = bnd & (lane == 63u ? ~0ull : ((2ull << lane) - 1ull));
    const uint32_t head = 63u - (uint32_t)__builtin_clzll(upto);
    const uint64_t after = head == 63u ? 0ull : bnd >> (head + 1u);
    const uint32_t end = after ? head + 1u + (uint32_t)__builtin_ctzll(after) : 64u;
    return KoRun{head, end - head, lane - head};
}

// Counts per major: one global atomic per run of equal majors in a wave
// (sorted input: about one per major; random input: about one per entry,
// which beats counting in LDS first when the majors far outnumber a block's
// entries).  KEY_NONE entries are not counted: their segment runs from the
// other majors' total to N.  They may fill most of the input (the final set's
// empty tile entries), and one counter taking an atomic per wave serializes,
// so k_ko_scatter places them with one atomic per block.
__global__ __launch_bounds__(256) void k_ko_count(const uint64_t *__restrict__ key, int64_t N, KeySplit ks,
                                                  uint32_t *__restrict__ cnt) {
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t m = e < N ? ks.major(key[e]) : 0xFFFFFFFFu;
    const KoRun r = ko_run(m, lane);
    if (m < ks.n_maj && r.rank == 0u) atomicAdd(cnt + m, r.len);
}

// ptr[0, n) = exclusive scan of cnt[0, n) (n <= KO_BINS), ptr[n] = n_all, by
// one block: the counts pass through LDS (coalesced loads and stores), thread t
// scans its KO_SCAN_PER consecutive ones (an odd stride: no bank conflicts),
// and a wave scan plus a scan over the 16 wave totals give its base.
constexpr uint32_t KO_SCAN_PER = (KO_BINS + 1023u) / 1024u;
__global__ __launch_bounds__(1024) void k_ko_scan(const uint32_t *__restrict__ cnt, uint32_t n, uint32_t n_all,
                                                  uint32_t *__restrict__ ptr) {
    __shared__ uint32_t wsum[16];
    __shared__ uint32_t sv[KO_SCAN_PER * 1024];
    const uint32_t t = threadIdx.x, lane = t & 63u, wave = t >> 6, b = t * KO_SCAN_PER;
#pragma unroll
    for (uint32_t k = 0; k < KO_SCAN_PER; ++k) {
        const uint32_t i = k * 1024u + t;
        sv[i] = i < n ? cnt[i] : 0u;
    }
    __syncthreads();
    uint32_t v[KO_SCAN_PER], s = 0;
#pragma unroll
    for (uint32_t k = 0; k < KO_SCAN_PER; ++k) {
        v[k] = sv[b + k];
        s += v[k];
    }
    uint32_t inc = s;
#pragma unroll
    for (uint32_t d = 1; d < 64u; d <<= 1) {
        const uint32_t o = (uint32_t)__shfl_up((int)inc, d, 64);
        if (lane >= d) inc += o;
    }
    if (lane == 63u) wsum[wave] = inc;
    __syncthreads();
    uint32_t base = 0;
#pragma unroll
    for (uint32_t w = 0; w < 16u; ++w) base += w < wave ? wsum[w] : 0u;
    uint32_t run = base + inc - s;
#pragma unroll
    for (uint32_t k = 0; k < KO_SCAN_PER; ++k) {
        sv[b + k] = run;
        run += v[k];
    }
    __syncthreads();
#pragma unroll
    for (uint32_t k = 0; k < KO_SCAN_PER; ++k) {
        const uint32_t i = k * 1024u + t;
        if (i < n) ptr[i] = sv[i];
    }
    if (t == 0) ptr[n] = n_all;  // the KEY_NONE segment (major n - 1, never counted) ends at n_all
}

// Each entry's place in its major's segment: ptr[m] plus the count left
// after its wave's run takes its share (cnt is consumed), plus its rank in the
// run.  KEY_NONE entries are final here: a block reserves its share of that
// segment by one atomic on none_fill, its waves' shares ranked in LDS.  Each
// thread takes KO_PER entries, 256 apart.
constexpr uint32_t KO_PER = 4, KO_CHUNK = 256 * KO_PER;
__global__ __launch_bounds__(256) void k_ko_scatter(const uint64_t *__restrict__ key, int64_t N, KeySplit ks,
                                                    const uint32_t *__restrict__ ptr, uint32_t *__restrict__ cnt,
                                                    uint32_t *__restrict__ none_fill,
                                                    uint32_t *__restrict__ seg_mnr, uint32_t *__restrict__ seg_idx,
                                                    uint64_t *__restrict__ key_out, uint32_t *__restrict__ perm) {
    __shared__ uint32_t s_none, s_base;
    if (threadIdx.x == 0) s_none = 0u;
    __syncthreads();
    const uint32_t lane = threadIdx.x & 63u;
    const int64_t e0 = (int64_t)blockIdx.x * KO_CHUNK + threadIdx.x;
    uint32_t noff[KO_PER];
#pragma unroll
    for (uint32_t k = 0; k < KO_PER; ++k) {
        const int64_t e = e0 + (int64_t)k * 256;
        const uint64_t kv = e < N ? key[e] : 0ull;
        const uint32_t m = e < N ? ks.major(kv) : 0xFFFFFFFFu;
        const KoRun r = ko_run(m, lane);
        uint32_t old = 0;
        if (m < ks.n_maj && r.rank == 0u) old = atomicSub(cnt + m, r.len);
        old = (uint32_t)__shfl((int)old, (int)r.head, 64);
        if (m < ks.n_maj) {
            const uint32_t p = ptr[m] + old - r.len + r.rank;
            seg_mnr[p] = ks.minor(kv);
            seg_idx[p] = (uint32_t)e;
        }
        const uint64_t none = __ballot(m == ks.n_maj);
        noff[k] = 0xFFFFFFFFu;
        if (none) {
            const uint32_t lead = (uint32_t)(__ffsll((unsigned long long)none) - 1);
            uint32_t o = 0;
            if (lane == lead) o = atomicAdd(&s_none, (uint32_t)__popcll(none));
            o = (uint32_t)__shfl((int)o, (int)lead, 64);
            if (m == ks.n_maj)
                noff[k] = o + __builtin_amdgcn_mbcnt_hi((uint32_t)(none >> 32),
                                                        __builtin_amdgcn_mbcnt_lo((uint32_t)none, 0u));
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) s_base = s_none ? ptr[ks.n_maj] + atomicAdd(none_fill, s_none) : 0u;
    __syncthreads();
    const uint32_t base = s_base;
#pragma unroll
    for (uint32_t k = 0; k < KO_PER; ++k) {
        if (noff[k] != 0xFFFFFFFFu) {
            const int64_t e = e0 + (int64_t)k * 256;
            key_out[base + noff[k]] = key[e];
            perm[base + noff[k]] = (uint32_t)e;
        }
    }
}

__device__ __forceinline__ uint64_t ko_pack(uint32_t mnr, uint32_t idx) { return ((uint64_t)mnr << 32) | idx; }

// One wave per major segment below n_maj; a segment longer than KO_CAP is
// listed for k_ko_long.
__global__ __launch_bounds__(KO_WAVES * 64) void k_ko_seg(const uint32_t *__restrict__ ptr, KeySplit ks,
                                                          const uint32_t *__restrict__ seg_mnr,
                                                          const uint32_t *__restrict__ seg_idx,
                                                          uint64_t *__restrict__ key_out, uint32_t *__restrict__ perm,
                                                          uint32_t *__restrict__ n_long, uint32_t *__restrict__ longs) {
    __shared__ uint64_t s[KO_WAVES][KO_CAP];
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const uint32_t m = blockIdx.x * KO_WAVES + wave;
    if (m >= ks.n_maj) return;
    const uint32_t b = ptr[m], len = ptr[m + 1] - b;
    if (len == 0u) return;
    if (len <= 64u) {
        // padding (all ones) sorts last: real pairs have idx < 2^31
        uint64_t v = lane < len ? ko_pack(seg_mnr[b + lane], seg_idx[b + lane]) : ~0ull;
        for (uint32_t k = 2; k <= 64u; k <<= 1)
            for (uint32_t j = k >> 1; j > 0; j >>= 1) {
                const uint32_t lo32 = (uint32_t)__shfl_xor((int)(uint32_t)v, (int)j, 64);
                const uint32_t hi32 = (uint32_t)__shfl_xor((int)(uint32_t)(v >> 32), (int)j, 64);
                const uint64_t o = ((uint64_t)hi32 << 32) | lo32;
                const bool up = (lane & k) == 0u, lower = (lane & j) == 0u;
                if (lower == up ? o < v : o > v) v = o;
            }
        if (lane < len) {
            key_out[b + lane] = ks.key(m, (uint32_t)(v >> 32));
            perm[b + lane] = (uint32_t)v;
        }
        return;
    }
    if (len > KO_CAP) {
        if (lane == 0) longs[atomicAdd(n_long, 1u)] = m;
        return;
    }
    uint32_t n2 = 128;
    while (n2 < len) n2 <<= 1;
    uint64_t *t = s[wave];
    for (uint32_t q = lane; q < n2; q += 64u) t[q] = q < len ? ko_pack(seg_mnr[b + q], seg_idx[b + q]) : ~0ull;
    wave_lds_sync();
    for (uint32_t k = 2; k <= n2; k <<= 1)
        for (uint32_t j = k >> 1; j > 0; j >>= 1) {
            for (uint32_t q = lane; q < n2 / 2u; q += 64u) {
                const uint32_t lo = (q / j) * 2u * j + (q % j), hi = lo + j;
                const bool up = (lo & k) == 0u;
                const uint64_t x = t[lo], y = t[hi];
                if (up ? x > y : x < y) {
                    t[lo] = y;
                    t[hi] = x;
                }
            }
            wave_lds_sync();
        }
    for (uint32_t q = lane; q < len; q += 64u) {
        const uint64_t v = t[q];
        key_out[b + q] = ks.key(m, (uint32_t)(v >> 32));
        perm[b + q] = (uint32_t)v;
    }
}

// The listed long segments, one block each: up to KO_LONG_LDS entries by a
// bitonic network in the block's LDS; beyond, in place in seg_mnr /
// seg_idx by a bitonic network whose comparators all put the smaller pair
// first (each merge starts by comparing mirrored positions), so positions at
// or past the segment's end act as +infinity and their comparators are
// skipped.  Rare: a major holding more than KO_CAP of the step's entries.
__global__ __launch_bounds__(256) void k_ko_long(const uint32_t *__restrict__ ptr, KeySplit ks,
                                                 const uint32_t *__restrict__ n_long,
                                                 const uint32_t *__restrict__ longs, uint32_t *seg_mnr,
                                                 uint32_t *seg_idx, uint64_t *__restrict__ key_out,
                                                 uint32_t *__restrict__ perm) {
    __shared__ uint64_t t[KO_LONG_LDS];
    const uint32_t nl = *n_long;
    for (uint32_t q = blockIdx.x; q < nl; q += gridDim.x) {
        const uint32_t m = longs[q], b = ptr[m], len = ptr[m + 1] - b;
        uint32_t *mn = seg_mnr + b, *ix = seg_idx + b;
        uint32_t n2 = 1;
        while (n2 < len) n2 <<= 1;
        if (len <= KO_LONG_LDS) {
            // the block's LDS: a plain bitonic network, padding sorting last
            for (uint32_t i = threadIdx.x; i < n2; i += 256u) t[i] = i < len ? ko_pack(mn[i], ix[i]) : ~0ull;
            __syncthreads();
            for (uint32_t k = 2; k <= n2; k <<= 1)
                for (uint32_t j = k >> 1; j > 0; j >>= 1) {
                    for (uint32_t i = threadIdx.x; i < n2 / 2u; i += 256u) {
                        const uint32_t lo = (i / j) * 2u * j + (i % j), hi = lo + j;
                        const bool up = (lo & k) == 0u;
                        const uint64_t x = t[lo], y = t[hi];
                        if (up ? x > y : x < y) {
                            t[lo] = y;
                            t[hi] = x;
                        }
                    }
                    __syncthreads();
                }
            for (uint32_t i = threadIdx.x; i < len; i += 256u) {
                key_out[b + i] = ks.key(m, (uint32_t)(t[i] >> 32));
                perm[b + i] = (uint32_t)t[i];
            }
            __syncthreads();
            continue;
        }
        for (uint32_t k = 2; k <= n2; k <<= 1)
            for (uint32_t j = k >> 1; j > 0; j >>= 1) {
                for (uint32_t t = threadIdx.x; t < n2 / 2u; t += 256u) {
                    const uint32_t lo = (t / j) * 2u * j + (t % j);
                    const uint32_t hi = j == (k >> 1) ? (lo / k) * k + (k - 1u) - (lo % k) : lo + j;
                    if (hi < len) {
                        const uint64_t x = ko_pack(mn[lo], ix[lo]), y = ko_pack(mn[hi], ix[hi]);
                        if (x > y) {
                            mn[lo] = (uint32_t)(y >> 32);
                            ix[lo] = (uint32_t)y;
                            mn[hi] = (uint32_t)(x >> 32);
                            ix[hi] = (uint32_t)x;
                        }
                    }
                }
                __syncthreads();
            }
        for (uint32_t t = threadIdx.x; t < len; t += 256u) {
            key_out[b + t] = ks.key(m, mn[t]);
            perm[b + t] = ix[t];
        }
        __syncthreads();
    }
}

// key_out = key[0, N) in order, perm = the entries' indices in that order
// (what a stable radix sort of (key, index) pairs gives).  False, with nothing
// launched, when the majors do not fit KO_BINS or N reaches 2^31: the caller
// sorts instead.  Set SILI_KEYORDER=0 to always sort.
bool order_keys(Layer &L, const uint64_t *key, int64_t N, uint32_t n_maj, uint64_t div, uint64_t *key_out,
                uint32_t *perm) {
    if (env_int("SILI_KEYORDER", 1) == 0 || (uint64_t)n_maj + 1u > KO_BINS || N >= (int64_t(1) << 31)) return false;
    if (N == 0) return true;
    hipStream_t st = L.stream;
    const KeySplit ks{div, n_maj};
    const uint32_t nb = n_maj + 1u;
    const int64_t max_long = N / (KO_CAP + 1) + 1;
    TmpBuf<uint32_t> cnt(L, SILI_TMPKEY(ko_cnt)), ptr(L, SILI_TMPKEY(ko_ptr)), smn(L, SILI_TMPKEY(ko_mnr)),
        sidx(L, SILI_TMPKEY(ko_idx)), longs(L, SILI_TMPKEY(ko_longs));
    cnt.ensure((size_t)nb + 2);  // [nb]: the long-segment count, [nb + 1]: KEY_NONE places taken
    ptr.ensure((size_t)nb + 1);
    smn.ensure((size_t)N);
    sidx.ensure((size_t)N);
    longs.ensure((size_t)max_long);
    launch(k_fill_u32, dim3(nblk(nb + 2)), dim3(TPB), 0, st, cnt.p, (int64_t)nb + 2, 0u);
    launch(k_ko_count, dim3((unsigned)((N + 255) / 256)), dim3(256), 0, st, key, N, ks, cnt.p);
    launch(k_ko_scan, dim3(1), dim3(1024), 0, st, (const uint32_t *)cnt.p, nb, (uint32_t)N, ptr.p);
    launch(k_ko_scatter, dim3((unsigned)((N + KO_CHUNK - 1) / KO_CHUNK)), dim3(256), 0, st, key, N, ks,
           (const uint32_t *)ptr.p, cnt.p, cnt.p + nb + 1, smn.p, sidx.p, key_out, perm);
    launch(k_ko_seg, dim3((n_maj + KO_WAVES - 1) / KO_WAVES), dim3(KO_WAVES * 64), 0, st, (const uint32_t *)ptr.p,
           ks, (const uint32_t *)smn.p, (const uint32_t *)sidx.p, key_out, perm, cnt.p + nb, longs.p);
    launch(k_ko_long, dim3((unsigned)std::min<int64_t>(max_long, KO_LONG_MAX_BLOCKS)), dim3(256), 0, st, (const uint32_t *)ptr.p, ks,
           (const uint32_t *)(cnt.p + nb), (const uint32_t *)longs.p, smn.p, sidx.p, key_out, perm);
    SILI_HIP(hipGetLastError());
    return true;
}

// Exclusive scan of flag[0, n) into pos; returns the total.  With n_mid:
// also the count of flags in [0, mid), read in the same round trip.
int64_t compact_positions(Layer &L, const uint32_t *flag, uint32_t *pos, int64_t n, int64_t mid = -1,
                          int64_t *n_mid = nullptr) {
    if (n == 0) {
        if (n_mid) *n_mid = 0;
        return 0;
    }
    device_exclusive_scan_u32(L, flag, pos, n);
    uint32_t last_pos = 0, last_flag = 0, at_mid = 0;
    ReadBack rb(L);
    rb.add(&last_pos, pos + n - 1, sizeof(uint32_t));
    rb.add(&last_flag, flag + n - 1, sizeof(uint32_t));
    const bool inner = n_mid && mid >= 0 && mid < n;
    if (inner) rb.add(&at_mid, pos + mid, sizeof(uint32_t));
    rb.wait();
    const int64_t total = (int64_t)last_pos + last_flag;
    if (n_mid) *n_mid = inner ? (int64_t)at_mid : total;
    return total;
}

template <typename K>
void sel_histogram(Layer &L, const K *keys, int64_t n, K limit, int shift, int width, int level,
                   const SelState *state, uint32_t *hist) {
    hipStream_t st = L.stream;
    const unsigned hb = (unsigned)std::min<int64_t>(1024, std::max<int64_t>(1, nblk(n)));
    launch(k_fill_u32, dim3(nblk(4096)), dim3(TPB), 0, st, hist, (int64_t)4096, 0u);
    launch(k_sel_hist<K>, dim3(hb), dim3(TPB), 0, st, keys, n, limit, shift, width, level, state, hist);
}

// Radix select over keys[0, n) below `limit` (bits significant bits): the
// state ends at the need-th smallest key (prefix), with `less` keys below it.
// have_level0: hist already holds the first level's histogram.
template <typename K>
void radix_select(Layer &L, const K *keys, int64_t n, K limit, int bits, SelState *state, uint32_t *hist,
                  bool have_level0 = false) {
    hipStream_t st = L.stream;
    int done = 0;
    for (int level = 0; done < bits; ++level) {
        const int width = std::min(12, bits - done);
        const int shift = bits - done - width;
        if (!(level == 0 && have_level0)) sel_histogram(L, keys, n, limit, shift, width, level, state, hist);
        launch(k_sel_find, dim3(1), dim3(TPB), 0, st, (const uint32_t *)hist, (uint32_t)(1u << width), width, state);
        done += width;
    }
    SILI_HIP(hipGetLastError());
}

// |w| bits of the live slots: 31 significant bits, dead slots 0xFFFFFFFF.
constexpr int ABSW_BITS = 31;
constexpr uint32_t ABSW_LIMIT = 0x80000000u;

// order[0, k) = the k live slots smallest by (|w| bits, row, col), in no
// particular order.  hist holds the first |w| level (count_live's).
void select_smallest(Layer &L, const uint32_t *absw, const uint64_t *rc, int64_t M, int64_t k, int rc_bits,
                     uint32_t *hist, uint32_t *order) {
    hipStream_t st = L.stream;
    TmpBuf<SelState> state(L, SILI_TMPKEY(state));
    state.ensure(2);
    const SelState s0{0ull, (unsigned long long)k, 0ull, 0ull};
    launch(k_put_state, dim3(1), dim3(1), 0, st, state.p, s0);
    radix_select<uint32_t>(L, absw, M, ABSW_LIMIT, ABSW_BITS, state.p, hist, true);
    const SelState sf = read_back(L, (const SelState *)state.p);
    const int64_t less = (int64_t)sf.less, ties = (int64_t)sf.pad, take = k - less;
    if ((int64_t)sf.need != take || take < 1 || take > ties)
        throw_error(SILI_ERR_RUNTIME, "synapto: selection of the smallest synapses is inconsistent");
    TmpBuf<uint32_t> tie_idx(L, SILI_TMPKEY(tie_idx)), tflag(L, SILI_TMPKEY(tflag)), tpos(L, SILI_TMPKEY(tpos));
    TmpBuf<uint64_t> tie_key(L, SILI_TMPKEY(tie_key));
    TmpBuf<uint64_t> bcnt(L, SILI_TMPKEY(bcnt)), boff(L, SILI_TMPKEY(boff));
    tie_idx.ensure((size_t)ties + 1);
    tie_key.ensure((size_t)ties + 1);
    const int64_t nb = nblk(M);
    bcnt.ensure((size_t)nb + 1);
    boff.ensure((size_t)nb + 1);
    launch(k_sel_count, dim3((unsigned)nb), dim3(TPB), 0, st, absw, M, (const SelState *)state.p, bcnt.p);
    SILI_HIP(hipGetLastError());
    device_exclusive_scan_u64(L, bcnt.p, boff.p, nb);
    launch(k_sel_place, dim3((unsigned)nb), dim3(TPB), 0, st, absw, rc, M, (const SelState *)state.p,
           (const uint64_t *)boff.p, order, tie_idx.p, tie_key.p);
    SILI_HIP(hipGetLastError());
    if (take == ties) {
        launch(k_copy_u32, dim3(nblk(take)), dim3(TPB), 0, st, (const uint32_t *)tie_idx.p, take, order + less);
        SILI_HIP(hipGetLastError());
        return;
    }
    // the first `take` ties in (row, col) order: keys up to the take-th smallest
    const SelState s1{0ull, (unsigned long long)take, 0ull, 0ull};
    launch(k_put_state, dim3(1), dim3(1), 0, st, state.p + 1, s1);
    radix_select<uint64_t>(L, tie_key.p, ties, ~0ull, rc_bits, state.p + 1, hist);
    tflag.ensure((size_t)ties + 1);
    tpos.ensure((size_t)ties + 1);
    launch(k_sel_tie_flags, dim3(nblk(ties + 1)), dim3(TPB), 0, st, (const uint64_t *)tie_key.p, ties,
           (const SelState *)(state.p + 1), tflag.p);
    device_exclusive_scan_u32(L, tflag.p, tpos.p, ties + 1);
    launch(k_sel_tie_scatter, dim3(nblk(ties)), dim3(TPB), 0, st, (const uint32_t *)tflag.p, (const uint32_t *)tpos.p,
           (const uint32_t *)tie_idx.p, ties, order + less);
    SILI_HIP(hipGetLastError());
}

}  // namespace

void synapto_step(Layer &L, float prune_frac, const int32_t *cand_r, const int32_t *cand_c,
                  const float *cand_v, const float *cand_s, int64_t n_cand, int default_imp,
                  int64_t *stats) {
    L.out_deg_tracked = false;  // a structure of this build's own policy: counted afresh
    // a layer that takes bulk steps keeps the step's temporaries (about 50
    // bytes per synapse slot) instead of allocating them every step, up to
    // 2^26 slots
    if (L.W.nnz + 16 * L.B4.ntiles < (int64_t(1) << 26)) L.keep_temps = true;
    synapto_apply(L, prune_frac, false, nullptr, 0, cand_r, cand_c, cand_v, cand_s, n_cand, default_imp, stats);
}

// The bulk pipeline.  explicit_prune false: prune the round(prune_frac * N)
// smallest |w| and regrow as many candidates.  True: prune exactly the
// n_prune stored synapses (row << 32 | col keys, host memory; none when
// n_prune is 0) and grow every valid candidate.
void synapto_apply(Layer &L, float prune_frac, bool explicit_prune, const uint64_t *prune_keys, int64_t n_prune,
                   const int32_t *cand_r, const int32_t *cand_c, const float *cand_v, const float *cand_s,
                   int64_t n_cand, int default_imp, int64_t *stats) {
    hipStream_t st = L.stream;
    const int64_t Ns = L.W.nnz, T = L.B4.ntiles;
    const int64_t n_in = L.n_in, n_out = L.n_out;
    const uint64_t bcols = (uint64_t)((n_out + 3) / 4);
    const int64_t M = Ns + 16 * T;  // synapse slots considered
    // radix-sort widths: (row << 32 | col) keys use 32 + bits(n_in) bits and
    // window keys bits(brows * bcols); every valid key then stays below the
    // low bits of KEY_NONE (all ones), which still sorts last
    auto bits_of = [](uint64_t v) {
        int b = 1;
        while (b < 64 && (v >> b) != 0) ++b;
        return b;
    };
    const int rc_bits = 32 + bits_of((uint64_t)n_in);
    const int win_bits = bits_of((uint64_t)((n_in + 3) / 4) * bcols);
    if (Ns + T + n_cand >= (int64_t(1) << 32) - 1 || M >= (int64_t(1) << 32) - 1)
        throw_error(SILI_ERR_RANGE, "synapto_step: layer too large for one step");
    const ScaleView sc = L.rank == 1
        ? ScaleView{L.vs_ones ? nullptr : L.vs.p, L.os_ones ? nullptr : L.os.p, 1}
        : ScaleView{L.vs.p, L.os.p, L.rank};

    // -- decode both stores --------------------------------------------------
    TmpBuf<uint32_t> srow(L, SILI_TMPKEY(srow)), scol(L, SILI_TMPKEY(scol)), tbr(L, SILI_TMPKEY(tbr)), tbc(L, SILI_TMPKEY(tbc));
    srow.ensure((size_t)Ns + 1);
    scol.ensure((size_t)Ns + 1);
    tbr.ensure((size_t)T + 1);
    tbc.ensure((size_t)T + 1);
    if (Ns > 0) decode_scattered(L, srow.p, scol.p);
    if (T > 0) launch_decode_b4(L.B4.plan(), tbr.p, tbc.p, st);
    TmpBuf<uint8_t> tbytes(L, SILI_TMPKEY(tbytes));  // tile bytes being edited (canonical order)
    tbytes.ensure((size_t)T * 16 + 1);
    if (T > 0) SILI_HIP(hipMemcpyAsync(tbytes.p, L.B4.tiles.p, (size_t)T * 16, hipMemcpyDeviceToDevice, st));
    TmpBuf<uint64_t> tkey(L, SILI_TMPKEY(tkey));  // window keys of the canonical tiles (ascending)
    tkey.ensure((size_t)T + 1);
    TmpBuf<uint8_t> tins(L, SILI_TMPKEY(tins));  // tiles that received an insert
    tins.ensure((size_t)T + 1);
    launch(k_fill_u8, dim3(nblk(T + 1)), dim3(TPB), 0, st, tins.p, T + 1, (uint8_t)0);

    // -- select: the k smallest by (|w| bits, row, col) ------------------------
    TmpBuf<uint64_t> rc(L, SILI_TMPKEY(rc)), rc_sorted(L, SILI_TMPKEY(rc_sorted));
    TmpBuf<uint32_t> absw(L, SILI_TMPKEY(absw)), iota(L, SILI_TMPKEY(iota)), perm_rc(L, SILI_TMPKEY(perm_rc)), order(L, SILI_TMPKEY(order));
    TmpBuf<unsigned long long> counters(L, SILI_TMPKEY(counters));  // live slots, demoted, grown
    TmpBuf<uint32_t> sel_hist(L, SILI_TMPKEY(sel_hist));
    counters.ensure(4);
    sel_hist.ensure(4096);
    rc.ensure((size_t)M + 1);
    absw.ensure((size_t)M + 1);
    order.ensure((size_t)M + 1);
    if (explicit_prune) {
        rc_sorted.ensure((size_t)M + 1);
        iota.ensure((size_t)M + 1);
        perm_rc.ensure((size_t)M + 1);
    }
    launch(k_fill_u32, dim3(1), dim3(TPB), 0, st, reinterpret_cast<uint32_t *>(counters.p), (int64_t)8, 0u);
    if (M > 0) {
        launch(k_syn_keys, dim3(nblk(M)), dim3(TPB), 0, st, Ns, (const uint32_t *)srow.p,
               (const uint32_t *)scol.p, (const uint8_t *)L.W.val.p, T, (const uint32_t *)tbr.p,
               (const uint32_t *)tbc.p, (const uint8_t *)L.B4.tiles.p, n_in, n_out, sc, rc.p, absw.p);
        SILI_HIP(hipGetLastError());
        if (!explicit_prune) {
            // the live slots: the first |w| level of the selection below
            sel_histogram<uint32_t>(L, absw.p, M, ABSW_LIMIT, ABSW_BITS - 12, 12, 0, nullptr, sel_hist.p);
            launch(k_hist_sum, dim3(1), dim3(TPB), 0, st, (const uint32_t *)sel_hist.p, 4096u, counters.p);
            SILI_HIP(hipGetLastError());
        } else {
            // (row, col) order: the explicit prune keys are looked up in it
            launch(k_iota32, dim3(nblk(M)), dim3(TPB), 0, st, iota.p, M);
            device_sort_pairs_u64(L, rc.p, rc_sorted.p, iota.p, perm_rc.p, M, rc_bits);
            launch(k_count_live, dim3(1), dim3(64), 0, st, (const uint64_t *)rc_sorted.p, M, counters.p);
            SILI_HIP(hipGetLastError());
        }
    }
    const int64_t N = (int64_t)read_back(L, counters.p);  // scattered + live block4 slots
    int64_t k = 0;
    if (explicit_prune) {
        if (n_prune > 0) {
            if (n_prune > M) throw_error(SILI_ERR_INVALID, "synapto: more prune keys than stored synapses");
            TmpBuf<uint64_t> dkeys(L, SILI_TMPKEY(dkeys));
            dkeys.ensure((size_t)n_prune);
            SILI_HIP(hipMemcpyAsync(dkeys.p, prune_keys, (size_t)n_prune * 8, hipMemcpyHostToDevice, st));
            L.scratch.flag.ensure(4, 0);
            SILI_HIP(hipMemsetAsync(L.scratch.flag.p, 0, 4 * sizeof(int), st));
            launch(k_find_slots, dim3(nblk(n_prune)), dim3(TPB), 0, st, (const uint64_t *)dkeys.p, n_prune,
                   (const uint64_t *)rc_sorted.p, (const uint32_t *)perm_rc.p, M, Ns, order.p, L.scratch.flag.p);
            SILI_HIP(hipGetLastError());
            int missing = 0;
            SILI_HIP(hipMemcpyAsync(&missing, L.scratch.flag.p, sizeof(int), hipMemcpyDeviceToHost, st));
            SILI_HIP(hipStreamSynchronize(st));
            if (missing) throw_error(SILI_ERR_RUNTIME, "synapto: a synapse to prune is not stored");
        }
        k = n_prune;
    } else {
        k = std::min<int64_t>(N, (int64_t)std::llround((double)prune_frac * (double)N));
        if (k > 0) select_smallest(L, absw.p, rc.p, M, k, rc_bits, sel_hist.p, order.p);
    }
    const int64_t k_grow = explicit_prune ? n_cand : k;  // candidates that may grow

    // -- prune ---------------------------------------------------------------
    TmpBuf<uint8_t> s_removed(L, SILI_TMPKEY(s_removed)), touched(L, SILI_TMPKEY(touched)), alive(L, SILI_TMPKEY(alive)), dem_byte(L, SILI_TMPKEY(dem_byte));
    TmpBuf<uint64_t> dem_key(L, SILI_TMPKEY(dem_key));
    s_removed.ensure((size_t)Ns + 1);
    touched.ensure((size_t)T + 1);
    alive.ensure((size_t)T + 1);
    dem_byte.ensure((size_t)T + 1);
    dem_key.ensure((size_t)T + 1);
    if (Ns > 0) launch(k_fill_u8, dim3(nblk(Ns)), dim3(TPB), 0, st, s_removed.p, Ns, (uint8_t)0);
    if (T > 0) launch(k_fill_u8, dim3(nblk(T)), dim3(TPB), 0, st, touched.p, T, (uint8_t)0);
    if (k > 0) {
        launch(k_syn_prune, dim3(nblk(k)), dim3(TPB), 0, st, (const uint32_t *)order.p, k, Ns, s_removed.p,
               tbytes.p, touched.p);
        SILI_HIP(hipGetLastError());
    }

    // -- demote --------------------------------------------------------------
    if (T > 0) {
        launch(k_syn_demote, dim3(nblk(T)), dim3(TPB), 0, st, T, (const uint32_t *)tbr.p,
               (const uint32_t *)tbc.p, (const uint8_t *)tbytes.p, (const uint8_t *)touched.p, n_in, n_out,
               alive.p, dem_key.p, dem_byte.p, counters.p + 1);
        SILI_HIP(hipGetLastError());
        // window keys of the canonical tiles, in store order (ascending)
        launch(k_tile_wkeys, dim3(nblk(T)), dim3(TPB), 0, st, (const uint32_t *)tbr.p, (const uint32_t *)tbc.p,
               T, bcols, tkey.p);
        SILI_HIP(hipGetLastError());
    }

    // -- scattered set after prune + demote -----------------------------------
    const int64_t M2 = Ns + T + n_cand;
    TmpBuf<uint64_t> key2(L, SILI_TMPKEY(key2)), key2_sorted(L, SILI_TMPKEY(key2_sorted));
    TmpBuf<uint8_t> byte2(L, SILI_TMPKEY(byte2)), byte2_sorted(L, SILI_TMPKEY(byte2_sorted)), removed2(L, SILI_TMPKEY(removed2));
    TmpBuf<uint32_t> iota2(L, SILI_TMPKEY(iota2)), perm2(L, SILI_TMPKEY(perm2));
    key2.ensure((size_t)M2 + 1);
    key2_sorted.ensure((size_t)M2 + 1);
    byte2.ensure((size_t)M2 + 1);
    byte2_sorted.ensure((size_t)M2 + 1);
    removed2.ensure((size_t)M2 + 1);
    iota2.ensure((size_t)M2 + 1);
    perm2.ensure((size_t)M2 + 1);
    if (Ns + T > 0) {
        launch(k_syn_set1, dim3(nblk(Ns + T)), dim3(TPB), 0, st, Ns, T, (const uint64_t *)rc.p,
               (const uint8_t *)L.W.val.p, (const uint8_t *)s_removed.p, (const uint64_t *)dem_key.p,
               (const uint8_t *)dem_byte.p, key2.p, byte2.p);
        SILI_HIP(hipGetLastError());
    }

    // -- candidates: first valid ones in list order ---------------------------
    TmpBuf<int32_t> dcr(L, SILI_TMPKEY(dcr)), dcc(L, SILI_TMPKEY(dcc));
    TmpBuf<float> dcv(L, SILI_TMPKEY(dcv)), dcs(L, SILI_TMPKEY(dcs));
    TmpBuf<uint64_t> ckey(L, SILI_TMPKEY(ckey)), ckey_sorted(L, SILI_TMPKEY(ckey_sorted)), win(L, SILI_TMPKEY(win)), win_sorted(L, SILI_TMPKEY(win_sorted));
    TmpBuf<uint32_t> cidx(L, SILI_TMPKEY(cidx)), cidx_sorted(L, SILI_TMPKEY(cidx_sorted)), first(L, SILI_TMPKEY(first)), rank(L, SILI_TMPKEY(rank)), wv(L, SILI_TMPKEY(wv)), wvs(L, SILI_TMPKEY(wvs));
    if (n_cand > 0) {
        dcr.ensure((size_t)n_cand);
        dcc.ensure((size_t)n_cand);
        dcv.ensure((size_t)n_cand);
        SILI_HIP(hipMemcpyAsync(dcr.p, cand_r, (size_t)n_cand * 4, hipMemcpyHostToDevice, st));
        SILI_HIP(hipMemcpyAsync(dcc.p, cand_c, (size_t)n_cand * 4, hipMemcpyHostToDevice, st));
        SILI_HIP(hipMemcpyAsync(dcv.p, cand_v, (size_t)n_cand * 4, hipMemcpyHostToDevice, st));
        if (cand_s) {
            dcs.ensure((size_t)n_cand);
            SILI_HIP(hipMemcpyAsync(dcs.p, cand_s, (size_t)n_cand * 4, hipMemcpyHostToDevice, st));
        }
        ckey.ensure((size_t)n_cand);
        ckey_sorted.ensure((size_t)n_cand);
        cidx.ensure((size_t)n_cand);
        cidx_sorted.ensure((size_t)n_cand);
        first.ensure((size_t)n_cand);
        rank.ensure((size_t)n_cand);
        win.ensure((size_t)n_cand);
        win_sorted.ensure((size_t)n_cand);
        wv.ensure((size_t)n_cand);
        wvs.ensure((size_t)n_cand);
        const unsigned g = nblk(n_cand);
        launch(k_syn_cand_static, dim3(g), dim3(TPB), 0, st, n_cand, (const int32_t *)dcr.p,
               (const int32_t *)dcc.p, n_in, n_out, (const uint64_t *)rc.p, Ns, (const uint64_t *)tkey.p, T,
               (const uint8_t *)L.B4.tiles.p, bcols, ckey.p);
        launch(k_fill_u32, dim3(g), dim3(TPB), 0, st, first.p, n_cand, 0u);
        SILI_HIP(hipGetLastError());
        if (!order_keys(L, ckey.p, n_cand, (uint32_t)n_in, 0, ckey_sorted.p, cidx_sorted.p)) {
            launch(k_iota32, dim3(g), dim3(TPB), 0, st, cidx.p, n_cand);
            device_sort_pairs_u64(L, ckey.p, ckey_sorted.p, cidx.p, cidx_sorted.p, n_cand, rc_bits);
        }
        launch(k_syn_first, dim3(g), dim3(TPB), 0, st, n_cand, (const uint64_t *)ckey_sorted.p,
               (const uint32_t *)cidx_sorted.p, first.p);
        SILI_HIP(hipGetLastError());
        device_exclusive_scan_u32(L, first.p, rank.p, n_cand);
        launch(k_syn_insert, dim3(g), dim3(TPB), 0, st, n_cand, (const uint32_t *)first.p,
               (const uint32_t *)rank.p, k_grow, (const int32_t *)dcr.p, (const int32_t *)dcc.p,
               (const float *)dcv.p, cand_s ? (const float *)dcs.p : nullptr, (uint32_t)default_imp, sc,
               (const uint64_t *)tkey.p, T, (const uint8_t *)alive.p, tbytes.p, tins.p, bcols, key2.p + (Ns + T),
               byte2.p + (Ns + T), win.p, counters.p + 2);
        SILI_HIP(hipGetLastError());
        if (!order_keys(L, win.p, n_cand, (uint32_t)((n_in + 3) / 4), bcols, win_sorted.p, wvs.p)) {
            launch(k_iota32, dim3(g), dim3(TPB), 0, st, wv.p, n_cand);
            device_sort_pairs_u64(L, win.p, win_sorted.p, wv.p, wvs.p, n_cand, win_bits);
        }
    }

    // -- final scattered set (sorted) and promotion ---------------------------
    if (M2 > 0) {
        launch(k_fill_u8, dim3(nblk(M2)), dim3(TPB), 0, st, removed2.p, M2, (uint8_t)0);
        SILI_HIP(hipGetLastError());
        if (!order_keys(L, key2.p, M2, (uint32_t)n_in, 0, key2_sorted.p, perm2.p)) {
            launch(k_iota32, dim3(nblk(M2)), dim3(TPB), 0, st, iota2.p, M2);
            device_sort_pairs_u64(L, key2.p, key2_sorted.p, iota2.p, perm2.p, M2, rc_bits);
        }
        launch(k_gather_u8_by, dim3(nblk(M2)), dim3(TPB), 0, st, (const uint8_t *)byte2.p,
               (const uint32_t *)perm2.p, M2, byte2_sorted.p);
        SILI_HIP(hipGetLastError());
    }
    TmpBuf<uint32_t> nt_flag(L, SILI_TMPKEY(nt_flag)), nt_br(L, SILI_TMPKEY(nt_br)), nt_bc(L, SILI_TMPKEY(nt_bc));
    TmpBuf<uint8_t> nt_bytes(L, SILI_TMPKEY(nt_bytes));
    nt_flag.ensure((size_t)n_cand + 1);
    nt_br.ensure((size_t)n_cand + 1);
    nt_bc.ensure((size_t)n_cand + 1);
    nt_bytes.ensure((size_t)n_cand * 16 + 1);
    if (n_cand > 0) {
        launch(k_syn_promote, dim3(nblk(n_cand)), dim3(TPB), 0, st, n_cand, (const uint64_t *)win_sorted.p,
               (const uint64_t *)key2_sorted.p, M2, (const uint8_t *)byte2_sorted.p, bcols, n_in,
               removed2.p, nt_flag.p, nt_br.p, nt_bc.p, nt_bytes.p);
        SILI_HIP(hipGetLastError());
    }

    // -- compaction + rebuild -------------------------------------------------
    TmpBuf<uint32_t> fflag(L, SILI_TMPKEY(fflag)), fpos(L, SILI_TMPKEY(fpos)), frows(L, SILI_TMPKEY(frows)), fcols(L, SILI_TMPKEY(fcols)), fptrs(L, SILI_TMPKEY(fptrs));
    TmpBuf<uint8_t> fbytes(L, SILI_TMPKEY(fbytes));
    fflag.ensure((size_t)M2 + 1);
    fpos.ensure((size_t)M2 + 1);
    if (M2 > 0) {
        launch(k_flag_final, dim3(nblk(M2)), dim3(TPB), 0, st, M2, (const uint64_t *)key2_sorted.p,
               (const uint8_t *)removed2.p, fflag.p);
        SILI_HIP(hipGetLastError());
    }
    const int64_t n_final = compact_positions(L, fflag.p, fpos.p, M2);
    frows.ensure((size_t)n_final + 1);
    fcols.ensure((size_t)n_final + 1);
    fbytes.ensure((size_t)n_final + 1);
    fptrs.ensure((size_t)n_in + 1);
    if (M2 > 0) {
        launch(k_emit_final, dim3(nblk(M2)), dim3(TPB), 0, st, M2, (const uint64_t *)key2_sorted.p,
               (const uint8_t *)byte2_sorted.p, (const uint32_t *)fflag.p, (const uint32_t *)fpos.p, frows.p,
               fcols.p, fbytes.p);
        SILI_HIP(hipGetLastError());
    }
    launch(k_row_ptrs, dim3(nblk(n_in + 1)), dim3(TPB), 0, st, (const uint32_t *)frows.p, n_final, n_in,
           fptrs.p);
    SILI_HIP(hipGetLastError());

    const int64_t MT = T + n_cand;
    TmpBuf<uint32_t> tflag(L, SILI_TMPKEY(tflag)), tpos(L, SILI_TMPKEY(tpos)), obr(L, SILI_TMPKEY(obr)), obc(L, SILI_TMPKEY(obc));
    TmpBuf<uint8_t> obytes(L, SILI_TMPKEY(obytes)), osparse(L, SILI_TMPKEY(osparse));
    tflag.ensure((size_t)MT + 1);
    tpos.ensure((size_t)MT + 1);
    if (MT > 0) {
        launch(k_tile_flags, dim3(nblk(MT)), dim3(TPB), 0, st, T, (const uint8_t *)alive.p, n_cand,
               (const uint32_t *)nt_flag.p, tflag.p);
        SILI_HIP(hipGetLastError());
    }
    // the surviving tiles come first, in store order, then the promoted
    // windows in window order: two runs of canonical order
    int64_t n_kept_tiles = 0;
    const int64_t n_tiles = compact_positions(L, tflag.p, tpos.p, MT, T, &n_kept_tiles);
    obr.ensure((size_t)n_tiles + 1);
    obc.ensure((size_t)n_tiles + 1);
    obytes.ensure((size_t)n_tiles * 16 + 1);
    osparse.ensure((size_t)n_tiles + 1);
    if (MT > 0) {
        launch(k_emit_tiles, dim3(nblk(MT)), dim3(TPB), 0, st, T, (const uint32_t *)tbr.p,
               (const uint32_t *)tbc.p, (const uint8_t *)tbytes.p, (const uint8_t *)L.B4.sparse.p,
               (const uint8_t *)tins.p, L.switch_point, n_cand, (const uint32_t *)nt_br.p,
               (const uint32_t *)nt_bc.p, (const uint8_t *)nt_bytes.p, (const uint32_t *)tflag.p,
               (const uint32_t *)tpos.p, obr.p, obc.p, obytes.p, osparse.p);
        SILI_HIP(hipGetLastError());
    }
    // both tile runs strictly increasing in (block row, block column)?  Read
    // back with the counters, before any store is replaced: a run out of
    // order (never expected) takes the full sort instead of the merge
    if (n_tiles > 1) {
        launch(k_tile_runs_order, dim3(nblk(n_tiles)), dim3(TPB), 0, st, (const uint32_t *)obr.p,
               (const uint32_t *)obc.p, n_tiles, n_kept_tiles, (uint64_t)bcols, counters.p + 3);
        SILI_HIP(hipGetLastError());
    }
    unsigned long long cnt[4];
    {
        ReadBack rb(L);
        rb.add(cnt, counters.p, sizeof(cnt));
        rb.wait();
    }
    // SILI_TILE_MERGE=0 always sorts (the two paths build the same store)
    const bool merge = cnt[3] == 0 && env_int("SILI_TILE_MERGE", 1) != 0;

    build_scattered(L, L.W, n_in, n_out, n_final, fptrs.p, fcols.p, fbytes.p);
    {
        struct Trusted {
            Layer &L;
            ~Trusted() { L.trusted_build = false; }
        } guard{L};
        L.trusted_build = true;
        build_shadow(L, L.W, frows.p, fcols.p, L.Wt);
        build_block4(L, n_tiles, obr.p, obc.p, obytes.p, osparse.p, merge ? n_kept_tiles : -1);
    }
    refresh_nonfinite(L);

    int64_t n_promoted = n_tiles - (T - (int64_t)cnt[1]);
    if (stats) {
        stats[0] = k;
        stats[1] = k;
        stats[2] = (int64_t)cnt[2];
        stats[3] = (int64_t)cnt[1];
        stats[4] = n_promoted;
        stats[5] = n_final;
        stats[6] = n_tiles;
    }
}

}  // namespace sili
