// policy.hip -- the reference's own synaptogenesis policy on the device store:
// delta_csr_build_probes (delta_csr_memory.hpp:1309-1426) and
// delta_csr_synap_row_step (delta_csr_memory.hpp:1021-1264).
//
// The policy is control logic over a handful of synapses per call (one row,
// k x k probes), so its decisions are made on the host from small reads of
// the device store (the block row being edited, staged into pinned memory in
// one round trip) with the same std::sort / std::partial_sort calls,
// comparators and input order as the reference -- its tie order is part of
// the result.
//
// The reference edits one synapse at a time: removals in descending column
// order, a block4 slot removal demoting its tile as soon as fewer than 2
// slots stay live; a later removal aimed at a slot that demotion moved to the
// scattered store finds no tile and does nothing.  The edits here run in
// phases (all removals, then demotion, inserts, promotion) as the bulk
// synaptogenesis pipeline runs them (synapto.hip), so the removals are first
// replayed on the block row's tiles and only those the reference performs
// are kept.  Inserts are equivalent either way: each insert's promotion check
// in the reference and one promotion pass leave the same tiles.  The block
// row's new state is computed here and written into the stores as a row
// patch (patch.hip); the bulk pipeline in its explicit-prune mode remains the
// path for what a patch does not cover (and SILI_POLICY_PATCH=0).
#include "../../include/sili_hip.h"
#include "layer.hpp"

#include <algorithm>
#include <array>
#include <map>
#include <numeric>
#include <set>
#include <unordered_set>
#include <vector>

namespace sili {

namespace {

constexpr unsigned TPB = 256;
inline unsigned nblk(int64_t n) { return (unsigned)((n + TPB - 1) / TPB); }

// out_degree before the policy's first step: the scattered synapses per
// column (the count the reference's load_weights keeps,
// sili/cpu_backend.cpp:446-447), i.e. the shadow store's row lengths.
__global__ void k_deg_from_starts(const uint32_t *__restrict__ t_elem_start, int64_t n_out, int32_t *deg) {
    const int64_t c = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (c < n_out) deg[c] = (int32_t)(t_elem_start[c + 1] - t_elem_start[c]);
}

// The policy's out_degree edits (delta_csr_memory.hpp:1216-1217,1246-1247):
// -1 (kept at >= 0) per removal entry, +1 per insert.  The columns of one
// call are distinct.
__global__ void k_deg_edit(int32_t *deg, const int32_t *__restrict__ cols, const int32_t *__restrict__ delta,
                           int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i >= n) return;
    const int32_t c = cols[i];
    if (delta[i] < 0) {
        if (deg[c] > 0) deg[c] -= 1;
    } else {
        deg[c] += 1;
    }
}
// The same for a short list carried in the arguments: col | 1 << 31 for a
// removal.
constexpr int DEG_INLINE = 256;
struct DegEdits {
    uint32_t n;
    uint32_t e[DEG_INLINE];
};
__global__ void k_deg_edit_inl(int32_t *deg, DegEdits d) {
    const uint32_t i = threadIdx.x;
    if (i >= d.n) return;
    const int32_t c = (int32_t)(d.e[i] & 0x7FFFFFFFu);
    if (d.e[i] >> 31) {
        if (deg[c] > 0) deg[c] -= 1;
    } else {
        deg[c] += 1;
    }
}

uint32_t uleb_read(const uint8_t *p, size_t &pos) {
    uint32_t v = 0;
    for (uint32_t sh = 0;; sh += 7) {
        const uint8_t b = p[pos++];
        v |= (uint32_t)(b & 0x7Fu) << sh;
        if (!(b & 0x80u)) return v;
    }
}

float fp4_value(uint32_t code) { return fp4_decode(code & 0xFu); }

// A staged canonical row as (col, (w<<4)|imp) in order.
std::vector<std::pair<uint32_t, uint8_t>> row_entries(const StagedRow &R) {
    const auto cols = staged_cols(R);
    std::vector<std::pair<uint32_t, uint8_t>> out(cols.size());
    for (size_t k = 0; k < cols.size(); ++k) out[k] = {cols[k], R.elems[k]};
    return out;
}

// Block rows as the policy sees them.  A block row the policy has edited is
// pending: its state lives here until policy_flush writes it.  Any other one
// is read from the device, STAGE_AHEAD block rows per round trip (the next
// calls' rows, as a sweep takes them), and kept as clean while no other
// entry point has run on the layer (policy_epoch).
constexpr uint32_t STAGE_AHEAD = 8;

StagedBlock block_from_staged(Layer &L, uint32_t br, StageReq &w, size_t w0, size_t nw, StageReq *b, size_t bj) {
    StagedBlock S;
    S.state.br = br;
    S.w.assign(w.out.begin() + (long)w0, w.out.begin() + (long)(w0 + nw));
    for (size_t l = 0; l < nw; ++l) S.state.rows[l] = row_entries(S.w[l]);
    S.has_b4 = b != nullptr;
    if (b) {
        S.b = b->out[bj];
        const auto bcs = staged_cols(S.b);
        for (size_t k = 0; k < bcs.size(); ++k) {
            PolicyTile t;
            std::copy(S.b.elems.begin() + k * 16, S.b.elems.begin() + k * 16 + 16, t.b.begin());
            t.sparse = S.b.flags[k];
            S.state.tiles[bcs[k]] = t;
        }
    }
    (void)L;
    return S;
}

// Requests staging block rows [br, br + n) that are neither pending nor
// clean (into `brs`), added to `reqs` (w: their canonical rows, b: their
// tiles).
void add_block_requests(Layer &L, uint32_t br, uint32_t n, StageReq &w, StageReq &b, std::vector<uint32_t> &brs) {
    const int64_t brows = (L.n_in + 3) / 4;
    const bool has_b4 = L.B4.byte_start.p != nullptr && L.B4.brows == brows;
    w.s = &L.W;
    b.b = &L.B4;
    b.flags = L.B4.sparse.p;
    for (uint32_t k = 0; k < n && (int64_t)(br + k) < brows; ++k) {
        const uint32_t q = br + k;
        if (L.policy_pending.count(q) || L.policy_clean.count(q)) continue;
        brs.push_back(q);
        for (int64_t r = (int64_t)q * 4; r < std::min<int64_t>((int64_t)q * 4 + 4, L.n_in); ++r)
            w.rows.push_back((uint32_t)r);
        if (has_b4) b.rows.push_back(q);
    }
    (void)has_b4;
}
// The staged rows into clean block rows.
void keep_clean(Layer &L, const std::vector<uint32_t> &brs, StageReq &w, StageReq &b) {
    size_t w0 = 0;
    for (size_t j = 0; j < brs.size(); ++j) {
        const uint32_t q = brs[j];
        const size_t nw = (size_t)(std::min<int64_t>((int64_t)q * 4 + 4, L.n_in) - (int64_t)q * 4);
        L.policy_clean[q] = block_from_staged(L, q, w, w0, nw, b.rows.empty() ? nullptr : &b, j);
        w0 += nw;
    }
}
void clean_valid(Layer &L) {
    if (L.clean_epoch != L.policy_epoch) {
        L.policy_clean.clear();
        L.clean_epoch = L.policy_epoch;
    }
}

// Block row br for a policy call, and whether it is pending.
StagedBlock &block_row(Layer &L, uint32_t br, BlockRowState *&cur) {
    auto p = L.policy_pending.find(br);
    if (p != L.policy_pending.end()) {
        cur = &p->second.cur;
        return p->second.orig;
    }
    clean_valid(L);
    auto c = L.policy_clean.find(br);
    if (c == L.policy_clean.end()) {
        StageReq w, b;
        std::vector<uint32_t> brs;
        add_block_requests(L, br, STAGE_AHEAD, w, b, brs);
        std::vector<StageReq *> reqs{&w};
        if (!b.rows.empty()) reqs.push_back(&b);
        stage_rows(L, reqs);
        keep_clean(L, brs, w, b);
        c = L.policy_clean.find(br);
    }
    cur = &c->second.state;
    return c->second;
}

inline uint8_t requant(uint32_t code) { return code == 8u ? 0u : (uint8_t)code; }

// The block row after the bulk pipeline's explicit-prune edit
// (synapto_apply): the removals (a scattered synapse, or with PRUNE_TILE a
// tile slot); every touched tile left with < 2 live slots demoted, its live slot
// becoming a scattered synapse with both nibbles requantized and swapped;
// the inserts of row li0 (weight 0, importance fp4(score)) into a surviving
// tile's slot, else scattered; every window that received a scattered insert
// and holds >= 2 scattered synapses promoted into a new tile.  A tile's
// tile_is_sparse is kept unless it received an insert or is new (then: live
// slots <= switch_point).
BlockRowState bulk_edit(const Layer &L, const BlockRowState &old, const std::vector<uint64_t> &prune_keys,
                        uint32_t li0, const std::vector<uint32_t> &add_cols, const std::vector<float> &add_scores,
                        int64_t no_promote = -1) {
    BlockRowState s = old;
    const int64_t r0 = (int64_t)s.br * 4;
    const uint32_t nr = (uint32_t)std::min<int64_t>(4, L.n_in - r0);
    auto find = [](std::vector<std::pair<uint32_t, uint8_t>> &row, uint32_t c) {
        return std::lower_bound(row.begin(), row.end(), std::make_pair(c, (uint8_t)0),
                                [](const std::pair<uint32_t, uint8_t> &a, const std::pair<uint32_t, uint8_t> &b) {
                                    return a.first < b.first;
                                });
    };
    auto put = [&](uint32_t li, uint32_t c, uint8_t byte) {
        auto &row = s.rows[li];
        auto it = find(row, c);
        if (it != row.end() && it->first == c) it->second = byte;
        else row.insert(it, {c, byte});
    };
    std::set<uint32_t> touched;
    for (uint64_t key : prune_keys) {
        const uint32_t li = (uint32_t)((int64_t)((key & ~PRUNE_TILE) >> 32) - r0), c = (uint32_t)(key & 0xFFFFFFFFu);
        if (!(key & PRUNE_TILE)) {
            auto &row = s.rows[li];
            auto it = find(row, c);
            if (it != row.end() && it->first == c) row.erase(it);
            continue;
        }
        auto t = s.tiles.find(c / 4);
        if (t != s.tiles.end()) {
            t->second.b[(c % 4) * 4 + li] = 0;
            touched.insert(c / 4);
        }
    }
    for (uint32_t bc : touched) {
        auto t = s.tiles.find(bc);
        int live = 0;
        for (uint8_t b : t->second.b) live += b != 0;
        if (live >= 2) continue;
        for (uint32_t sl = 0; sl < 16; ++sl) {
            const uint32_t b = t->second.b[sl], li = sl & 3u, c = bc * 4 + (sl >> 2);
            if (b == 0 || li >= nr || (int64_t)c >= L.n_out) continue;
            put(li, c, (uint8_t)((requant(b & 0xFu) << 4) | requant(b >> 4)));
        }
        s.tiles.erase(t);
    }
    std::set<uint32_t> windows, tins;
    for (size_t i = 0; i < add_cols.size(); ++i) {
        const uint32_t c = add_cols[i], bc = c / 4;
        const uint32_t ic = fp4_encode(add_scores[i]);  // the weight's code is fp4(0 / S) = 0
        auto t = s.tiles.find(bc);
        if (t != s.tiles.end()) {
            t->second.b[(c % 4) * 4 + li0] = (uint8_t)(ic << 4);
            tins.insert(bc);
        } else {
            put(li0, c, (uint8_t)ic);
            windows.insert(bc);
        }
    }
    for (uint32_t bc : windows) {
        if ((int64_t)bc == no_promote) continue;
        std::vector<std::pair<uint32_t, std::pair<uint32_t, uint8_t>>> found;  // (li, (c, byte))
        for (uint32_t li = 0; li < nr; ++li)
            for (auto it = find(s.rows[li], bc * 4); it != s.rows[li].end() && it->first < bc * 4 + 4; ++it)
                found.push_back({li, *it});
        if (found.size() < 2) continue;
        PolicyTile nt;
        for (const auto &f : found) {
            const uint32_t c = f.second.first, b = f.second.second;
            nt.b[(c - bc * 4) * 4 + f.first] = (uint8_t)(requant(b >> 4) | (requant(b & 0xFu) << 4));
            auto &row = s.rows[f.first];
            row.erase(find(row, c));
        }
        uint32_t live = 0;
        for (uint8_t b : nt.b) live += b != 0;
        nt.sparse = live <= L.switch_point ? 1 : 0;
        s.tiles[bc] = nt;
    }
    for (uint32_t bc : tins) {
        auto t = s.tiles.find(bc);
        if (t == s.tiles.end()) continue;
        uint32_t live = 0;
        for (uint8_t b : t->second.b) live += b != 0;
        t->second.sparse = live <= L.switch_point ? 1 : 0;
    }
    return s;
}

inline uint64_t uleb_len(uint32_t v) {
    uint64_t n = 1;
    while (v >= 0x80u) {
        v >>= 7;
        ++n;
    }
    return n;
}

// The four rows of one block row and its tiles, edited one synapse at a time
// as the reference edits its store in place: the rows' columns and index
// bytes, checked against the rows' reservations (L.lay_b, L.lay_e) the way
// delta_csr_row_insert_col (delta_csr_memory.hpp:498-585) checks them.
struct BlockRowSim {
    struct Row {
        std::vector<uint32_t> cols;  // ascending
        uint64_t bytes = 0;          // ULEB128 bytes of the row's deltas
        bool loaded = false;
    };
    Layer &L;
    uint32_t br;
    std::map<uint32_t, std::array<uint8_t, 16>> &tiles;
    Row rows[4];

    // rows past n_in stay empty; every other row is set from the staged block row
    Row &row(uint32_t li) {
        Row &R = rows[li];
        R.loaded = true;
        return R;
    }
    void set(uint32_t li, const std::vector<std::pair<uint32_t, uint8_t>> &entries) {
        Row &R = rows[li];
        R.cols.clear();
        R.bytes = 0;
        uint32_t prev = 0;
        for (const auto &e : entries) {
            R.cols.push_back(e.first);
            R.bytes += uleb_len(e.first - prev);
            prev = e.first;
        }
        R.loaded = true;
    }
    // false: the column is stored already, or does not fit the reservation
    bool insert(uint32_t li, uint32_t c) {
        Row &R = row(li);
        const size_t r = (size_t)br * 4 + li;
        auto it = std::lower_bound(R.cols.begin(), R.cols.end(), c);
        if (it != R.cols.end() && *it == c) return false;
        const uint32_t prev = it == R.cols.begin() ? 0u : *(it - 1);
        uint64_t grow = uleb_len(c - prev), shrink = 0;
        if (it != R.cols.end()) {
            grow += uleb_len(*it - c);
            shrink = uleb_len(*it - prev);
        }
        const int64_t idx_delta = (int64_t)grow - (int64_t)shrink;
        // unsigned as the reference evaluates it
        if (idx_delta > 0 && (uint64_t)idx_delta > L.lay_b[r] - R.bytes) return false;
        if ((uint64_t)R.cols.size() >= L.lay_e[r]) return false;
        R.cols.insert(it, c);
        R.bytes = (uint64_t)((int64_t)R.bytes + idx_delta);
        return true;
    }
    void remove(uint32_t li, uint32_t c) {
        Row &R = row(li);
        auto it = std::lower_bound(R.cols.begin(), R.cols.end(), c);
        if (it == R.cols.end() || *it != c) return;
        const uint32_t prev = it == R.cols.begin() ? 0u : *(it - 1);
        uint64_t freed = uleb_len(c - prev), merged = 0;
        if (it + 1 != R.cols.end()) {
            freed += uleb_len(*(it + 1) - c);
            merged = uleb_len(*(it + 1) - prev);
        }
        R.bytes = R.bytes - freed + merged;
        R.cols.erase(it);
    }
    // block4_maybe_promote (delta_csr_memory.hpp:591-702) after an insert at
    // (row li, column c): into the window's tile, or a new tile when the
    // window's four rows hold >= 2 scattered synapses
    void promote(uint32_t li, uint32_t c) {
        const uint32_t bc = c / 4;
        auto t = tiles.find(bc);
        if (t != tiles.end()) {
            t->second[(c % 4) * 4 + li] = 1;
            remove(li, c);
            return;
        }
        std::vector<std::pair<uint32_t, uint32_t>> found;
        for (uint32_t l = 0; l < 4 && (int64_t)br * 4 + l < L.n_in; ++l)
            for (uint32_t col : row(l).cols)
                if (col / 4 == bc) found.push_back({l, col});
        if (found.size() < 2) return;
        std::array<uint8_t, 16> d{};
        for (const auto &f : found) d[(f.second % 4) * 4 + f.first] = 1;
        tiles[bc] = d;
        for (const auto &f : found) remove(f.first, f.second);
    }
};

// The block4 store's reservations under one synap_row_step
// (delta_csr_memory.hpp:1203-1258), replayed edit by edit on block row br as
// the reference makes them: a tile slot's removal through a handle (a
// sparse tile re-committed, a dense one written in place), a demotion's
// erase, and each insert's promotion -- a write into an existing tile
// (committed when sparse, then maybe_compress) or a new tile
// (get_or_create: the row grown without room, the budget's MemoryError;
// then the commit of its slots).  A commit dropped at the tile budget
// leaves its tile as it was (counted in L.b4_dropped); such tiles are
// returned with their final bytes, which the call's new state takes.  When
// a new tile's row growth meets the budget, *nomem_at is set to that
// insert's index (its scattered insert stands, its window is not promoted,
// later inserts are not made).
struct B4Replay {
    std::map<uint32_t, PolicyTile> dropped;  // tiles whose commit was dropped: their final state
    int64_t nomem_at = -1;
    uint32_t nomem_bc = 0;
    std::string nomem_msg;
};

B4Replay b4_policy_replay(Layer &L, const BlockRowState &state, uint32_t li, const std::vector<uint32_t> &rm_cols,
                          const std::vector<bool> &rm_is_b4, const std::vector<uint32_t> &add_cols,
                          const std::vector<float> &add_scores) {
    B4Replay out;
    const size_t br = state.br;
    const uint32_t nr = (uint32_t)std::min<int64_t>(4, L.n_in - (int64_t)br * 4);
    std::map<uint32_t, PolicyTile> tiles = state.tiles;
    std::map<uint32_t, uint8_t> rows[4];
    for (uint32_t l = 0; l < 4; ++l)
        for (const auto &e : state.rows[l]) rows[l][e.first] = e.second;
    std::set<uint32_t> touched_by_drop;
    auto live_of = [](const PolicyTile &t) {
        uint32_t n = 0;
        for (uint8_t b : t.b) n += b != 0;
        return n;
    };
    auto len_of = [&](const PolicyTile &t) { return (uint64_t)tile_len(t.sparse != 0, live_of(t)); };
    auto use = [&](uint64_t &ui, uint64_t &ue, uint64_t &ut) {
        ui = ue = ut = 0;
        uint32_t prev = 0;
        for (const auto &kv : tiles) {
            ui += uleb_len(kv.first - prev);
            prev = kv.first;
            ++ue;
            ut += len_of(kv.second);
        }
    };
    // a sparse tile's handle commits its slots re-encoded by live count; a
    // dense one is written in place.  false: the commit was dropped
    auto write_slot = [&](uint32_t bc, uint32_t slot, uint8_t byte) {
        PolicyTile &t = tiles[bc];
        if (!t.sparse) {
            t.b[slot] = byte;
            return true;
        }
        uint64_t ui, ue, ut;
        use(ui, ue, ut);
        PolicyTile nt = t;
        nt.b[slot] = byte;
        const uint32_t live = live_of(nt);
        nt.sparse = live <= L.switch_point ? 1 : 0;
        if (!b4res_commit(L, br, len_of(t), len_of(nt), ut)) {
            touched_by_drop.insert(bc);
            return false;
        }
        t = nt;
        return true;
    };
    for (size_t k = 0; k < rm_cols.size(); ++k) {
        const uint32_t c = rm_cols[k];
        if (!rm_is_b4[k]) {
            rows[li].erase(c);
            continue;
        }
        auto it = tiles.find(c / 4);
        const uint32_t slot = (c % 4) * 4 + li;
        if (it == tiles.end() || it->second.b[slot] == 0) continue;
        write_slot(c / 4, slot, 0);
        it = tiles.find(c / 4);
        if (live_of(it->second) < 2) {  // block4_demote_tile, then the tile's erase
            const uint32_t bc = it->first;
            for (uint32_t sl = 0; sl < 16; ++sl) {
                const uint32_t b = it->second.b[sl], l2 = sl & 3u, c2 = bc * 4 + (sl >> 2);
                if (b == 0 || l2 >= nr || (int64_t)c2 >= L.n_out) continue;
                rows[l2][c2] = (uint8_t)((requant(b & 0xFu) << 4) | requant(b >> 4));
            }
            tiles.erase(it);
        }
    }
    for (size_t i = 0; i < add_cols.size(); ++i) {
        const uint32_t c = add_cols[i], bc = c / 4;
        rows[li][c] = (uint8_t)fp4_encode(add_scores[i]);  // weight code fp4(0) = 0
        auto it = tiles.find(bc);
        if (it != tiles.end()) {
            const uint8_t sb = rows[li][c];
            write_slot(bc, (c % 4) * 4 + li, (uint8_t)(requant(sb >> 4) | (requant(sb & 0xFu) << 4)));
            PolicyTile &t = tiles[bc];
            if (!t.sparse && live_of(t) <= L.switch_point) t.sparse = 1;  // maybe_compress
            rows[li].erase(c);
            continue;
        }
        std::vector<std::pair<uint32_t, uint32_t>> found;  // (row in block, column)
        for (uint32_t l = 0; l < nr; ++l)
            for (auto e = rows[l].lower_bound(bc * 4); e != rows[l].end() && e->first < bc * 4 + 4; ++e)
                found.push_back({l, e->first});
        if (found.size() < 2) continue;
        uint64_t ui, ue, ut;
        use(ui, ue, ut);
        auto nx = tiles.upper_bound(bc);
        const uint32_t prev = nx == tiles.begin() ? 0u : std::prev(nx)->first;
        int64_t d = (int64_t)uleb_len(bc - prev);
        if (nx != tiles.end()) d += (int64_t)uleb_len(nx->first - bc) - (int64_t)uleb_len(nx->first - prev);
        try {
            b4res_insert_tile(L, br, d, ui, ue, ut);
        } catch (const Error &e) {
            out.nomem_at = (int64_t)i;
            out.nomem_bc = bc;
            out.nomem_msg = e.msg;
            break;
        }
        PolicyTile nt;
        nt.sparse = 1;  // new tiles start sparse-empty (1 byte)
        tiles[bc] = nt;
        PolicyTile full = nt;
        for (const auto &f : found) {
            const uint8_t sb = rows[f.first][f.second];
            full.b[(f.second - bc * 4) * 4 + f.first] = (uint8_t)(requant(sb >> 4) | (requant(sb & 0xFu) << 4));
        }
        full.sparse = live_of(full) <= L.switch_point ? 1 : 0;
        if (b4res_commit(L, br, 1, len_of(full), ut + 1)) tiles[bc] = full;
        else touched_by_drop.insert(bc);
        for (const auto &f : found) rows[f.first].erase(f.second);
    }
    for (uint32_t bc : touched_by_drop) {
        auto it = tiles.find(bc);
        if (it != tiles.end()) out.dropped[bc] = it->second;
    }
    return out;
}

// L.out_deg holds out_degree; mark: from now on the policy keeps it.
void ensure_out_deg(Layer &L, bool mark) {
    if (L.out_deg_tracked) return;
    L.out_deg.ensure((size_t)std::max<int64_t>(1, L.n_out));
    if (L.n_out > 0)
        launch(k_deg_from_starts, dim3(nblk(L.n_out)), dim3(TPB), 0, L.stream, (const uint32_t *)L.Wt.elem_start.p,
               L.n_out, L.out_deg.p);
    SILI_HIP(hipGetLastError());
    L.out_deg_tracked = mark;
}

}  // namespace

void build_probes(Layer &L, int64_t k, bool per_row) {
    const size_t n_in = (size_t)L.n_in, n_out = (size_t)L.n_out;
    if (n_in == 0 || n_out == 0 || k <= 0) {
        L.probe_nnz = 0;  // the reference zeroes the count only
        return;
    }
    L.keep_temps = true;  // a layer that runs the policy keeps its small temporaries
    const float *acc_in = stage_accumulators(L), *acc_grad = acc_in + n_in;
    const size_t kk_in = std::min((size_t)k, n_in), kk = (size_t)k;
    if (L.sel_in_k != k) {  // the top rows, kept with the staged accumulators
        std::vector<size_t> in_idx(n_in);
        std::iota(in_idx.begin(), in_idx.end(), 0);
        std::partial_sort(in_idx.begin(), in_idx.begin() + kk_in, in_idx.end(),
                          [&](size_t a, size_t b) { return acc_in[a] > acc_in[b]; });
        in_idx.resize(kk_in);
        L.sel_in.swap(in_idx);
        L.sel_in_k = k;
    }
    const std::vector<size_t> &in_idx = L.sel_in;
    std::vector<int32_t> pr, pc;
    std::vector<float> pv;
    // the top rows' stored columns (edited block rows from their pending
    // state), staged in one round trip with the block row the next
    // synap_step edits
    clean_valid(L);
    {
        std::set<uint32_t> want;
        for (size_t r : in_idx) {
            const uint32_t q = (uint32_t)(r / 4);
            if (!L.policy_pending.count(q) && !L.policy_clean.count(q)) want.insert(q);
        }
        // the next synap_step's (a sweep's later calls stage theirs ahead)
        const uint32_t next_br = (uint32_t)((L.synap_cursor % L.n_in) / 4);
        if (!L.policy_pending.count(next_br) && !L.policy_clean.count(next_br)) want.insert(next_br);
        StageReq w, b;
        std::vector<uint32_t> brs;
        for (uint32_t q : want) add_block_requests(L, q, 1, w, b, brs);
        if (!brs.empty()) {
            std::vector<StageReq *> reqs{&w};
            if (!b.rows.empty()) reqs.push_back(&b);
            stage_rows(L, reqs);
            keep_clean(L, brs, w, b);
        }
    }
    auto row_cols = [&](size_t r) {
        const uint32_t q = (uint32_t)(r / 4);
        auto p = L.policy_pending.find(q);
        const BlockRowState &st = p != L.policy_pending.end() ? p->second.cur : L.policy_clean.at(q).state;
        std::vector<uint32_t> cols;
        for (const auto &e : st.rows[r % 4]) cols.push_back(e.first);
        return cols;
    };
    if (!per_row) {
        const size_t kk_out = std::min(kk, n_out);
        if (L.sel_out_k != k) {
            std::vector<size_t> out_idx(n_out);
            std::iota(out_idx.begin(), out_idx.end(), 0);
            std::partial_sort(out_idx.begin(), out_idx.begin() + kk_out, out_idx.end(),
                              [&](size_t a, size_t b) { return acc_grad[a] > acc_grad[b]; });
            out_idx.resize(kk_out);
            L.sel_out.swap(out_idx);
            L.sel_out_k = k;
        }
        const std::vector<size_t> &out_idx = L.sel_out;
        for (size_t r : in_idx) {
            const auto ex = row_cols(r);
            for (size_t c : out_idx) {
                if (std::binary_search(ex.begin(), ex.end(), (uint32_t)c)) continue;
                pr.push_back((int32_t)r);
                pc.push_back((int32_t)c);
                pv.push_back(acc_in[r] * acc_grad[c]);
            }
        }
    } else {
        for (size_t r : in_idx) {
            const auto ex = row_cols(r);
            std::vector<size_t> cand;
            cand.reserve(n_out);
            for (size_t c = 0; c < n_out; ++c)
                if (!std::binary_search(ex.begin(), ex.end(), (uint32_t)c)) cand.push_back(c);
            const size_t kk_row = std::min(kk, cand.size());
            if (kk_row == 0) continue;
            std::partial_sort(cand.begin(), cand.begin() + kk_row, cand.end(),
                              [&](size_t a, size_t b) { return acc_grad[a] > acc_grad[b]; });
            for (size_t i = 0; i < kk_row; ++i) {
                pr.push_back((int32_t)r);
                pc.push_back((int32_t)cand[i]);
                pv.push_back(acc_in[r] * acc_grad[cand[i]]);
            }
        }
    }
    L.probe_r.swap(pr);
    L.probe_c.swap(pc);
    L.probe_v.swap(pv);
    L.probe_nnz = (int64_t)L.probe_r.size();
}

bool synap_row_step(Layer &L, int64_t &cursor, float importance_cutoff, int64_t max_row_weights,
                    int64_t max_prune_per_step, float importance_eps) {
    if (L.n_in == 0) return false;
    L.keep_temps = true;  // a layer that runs the policy rebuilds often: keep the rebuild's temporaries
    if (L.lay_b.size() != (size_t)L.n_in) {
        policy_flush(L);  // the reservations fit the device's rows
        layout_fit(L);
    }
    const int64_t cursor0 = cursor;
    const int64_t row = cursor % L.n_in;
    cursor = (cursor + 1) % L.n_in;
    const uint32_t br = (uint32_t)(row / 4), li = (uint32_t)(row % 4);
    const int patch_mode = env_int("SILI_POLICY_PATCH", 1), defer = env_int("SILI_POLICY_DEFER", 1);
    if (!(patch_mode && defer) && !L.policy_pending.empty()) policy_flush(L);
    BlockRowState *curp = nullptr;
    StagedBlock &SB = block_row(L, br, curp);
    const BlockRowState state = *curp;  // the block row as the edits find it
    const auto &scat = state.rows[li];
    std::map<uint32_t, std::array<uint8_t, 16>> btiles;
    for (const auto &t : state.tiles) btiles[t.first] = t.second.b;
    std::vector<uint32_t> exist_cols;
    std::vector<float> exist_imp;
    std::vector<bool> exist_is_b4;
    for (const auto &e : scat) {
        exist_cols.push_back(e.first);
        exist_imp.push_back(fp4_value(e.second));
        exist_is_b4.push_back(false);
    }
    for (const auto &t : btiles)
        for (uint32_t lj = 0; lj < 4; ++lj) {
            const uint8_t b = t.second[lj * 4 + li];
            const uint32_t col = t.first * 4 + lj;
            if (b == 0 || col >= (uint32_t)L.n_out) continue;
            exist_cols.push_back(col);
            exist_imp.push_back(fp4_value(b >> 4));
            exist_is_b4.push_back(true);
        }
    const size_t n_exist = exist_cols.size();
    const bool has_probes = !L.probe_r.empty();
    if (n_exist == 0 && !has_probes) return false;
    std::vector<uint32_t> probe_cols;
    std::vector<float> probe_scores;
    for (int64_t p = 0; p < L.probe_nnz; ++p)
        if ((int64_t)L.probe_r[(size_t)p] == row) {
            probe_cols.push_back((uint32_t)L.probe_c[(size_t)p]);
            probe_scores.push_back(L.probe_v[(size_t)p]);
        }
    // removals: lowest importance first, below the cutoff (importance floored
    // at eps for this test only) or beyond the row's capacity, at most
    // max_prune_per_step of them; applied in descending column order
    std::vector<size_t> by_imp(n_exist);
    std::iota(by_imp.begin(), by_imp.end(), 0);
    std::sort(by_imp.begin(), by_imp.end(), [&](size_t a, size_t b) { return exist_imp[a] < exist_imp[b]; });
    struct Removal { uint32_t col; bool is_b4; };
    std::vector<Removal> to_remove;
    const size_t max_rw = (size_t)max_row_weights, max_prune = (size_t)max_prune_per_step;
    for (size_t rank = 0; rank < n_exist && to_remove.size() < max_prune; ++rank) {
        const size_t k = by_imp[rank];
        const size_t keep = n_exist - to_remove.size();
        if (std::max(exist_imp[k], importance_eps) < importance_cutoff || keep > max_rw)
            to_remove.push_back({exist_cols[k], exist_is_b4[k]});
    }
    std::sort(to_remove.begin(), to_remove.end(), [](const Removal &a, const Removal &b) { return a.col > b.col; });
    // inserts: the row's probes by descending score that are not stored, up
    // to the capacity the removals leave (unsigned, as the reference computes it)
    std::vector<uint32_t> add_cols;
    std::vector<float> add_scores;
    {
        std::unordered_set<uint32_t> exist_set(exist_cols.begin(), exist_cols.end());
        std::vector<size_t> pidx(probe_cols.size());
        std::iota(pidx.begin(), pidx.end(), 0);
        std::sort(pidx.begin(), pidx.end(), [&](size_t a, size_t b) { return probe_scores[a] > probe_scores[b]; });
        const size_t slots = max_rw - (n_exist - to_remove.size());
        for (size_t p : pidx) {
            if (add_cols.size() >= slots) break;
            if (!exist_set.count(probe_cols[p])) {
                add_cols.push_back(probe_cols[p]);
                add_scores.push_back(probe_scores[p]);
            }
        }
    }
    // replay the call's edits as the reference makes them, one synapse at a
    // time: which removals it carries out, and whether every slot a demotion
    // moves back to its row and every insert fits the row's reservation
    BlockRowSim sim{L, br, btiles, {}};
    for (uint32_t l = 0; l < (uint32_t)SB.w.size(); ++l) sim.set(l, state.rows[l]);
    std::vector<uint64_t> prune_keys;
    for (const auto &re : to_remove) {
        if (re.is_b4) {
            auto it = btiles.find(re.col / 4);
            const uint32_t s = (re.col % 4) * 4 + li;
            if (it == btiles.end() || it->second[s] == 0) continue;
            it->second[s] = 0;
            prune_keys.push_back(((uint64_t)row << 32) | re.col | PRUNE_TILE);
            int live = 0;
            for (uint8_t b : it->second) live += b != 0;
            if (live < 2) {  // block4_demote_tile: the slot left goes back to its row
                const uint32_t bc = it->first;
                for (uint32_t l2 = 0; l2 < 4; ++l2)
                    for (uint32_t j2 = 0; j2 < 4; ++j2) {
                        const int64_t r2 = (int64_t)br * 4 + l2, c2 = (int64_t)bc * 4 + j2;
                        if (it->second[j2 * 4 + l2] == 0 || r2 >= L.n_in || c2 >= L.n_out) continue;
                        if (!sim.insert(l2, (uint32_t)c2)) {
                            cursor = cursor0;
                            throw_error(SILI_ERR_RUNTIME,
                                        "block4_demote_tile: row " + std::to_string(r2) +
                                            " ran out of blank space while demoting tile (" + std::to_string(br) +
                                            "," + std::to_string(bc) +
                                            "). Call equalizer_step() to redistribute space from adjacent rows "
                                            "before retrying.");
                        }
                    }
                btiles.erase(it);
            }
        } else {
            prune_keys.push_back(((uint64_t)row << 32) | re.col);
            sim.remove(li, re.col);
        }
    }
    // the inserts, each followed by the promotion check; the first one that
    // does not fit ends the call (delta_csr_memory.hpp:1236-1250) with the
    // removals and the inserts before it applied
    std::string no_room;
    for (size_t i = 0; i < add_cols.size(); ++i) {
        if (!sim.insert(li, add_cols[i])) {
            no_room = "delta_csr_synap_row_step: row " + std::to_string(row) + " ran out of blank space at probe_index=" +
                      std::to_string(i) + " col=" + std::to_string(add_cols[i]) + " (used " +
                      std::to_string(sim.row(li).bytes) + " / " + std::to_string(L.lay_b[(size_t)row]) + " bytes, " +
                      std::to_string(add_cols.size() - i) +
                      " insertions skipped). Call equalizer_step() to redistribute space from adjacent rows before "
                      "retrying, or reduce max_row_weights / raise importance_cutoff.";
            add_cols.resize(i);
            add_scores.resize(i);
            break;
        }
        sim.promote(li, add_cols[i]);
    }
    // the block4 store's reservations under these edits
    B4Replay b4r;
    {
        std::vector<uint32_t> rm_cols;
        std::vector<bool> rm_b4;
        for (const auto &re : to_remove) {
            rm_cols.push_back(re.col);
            rm_b4.push_back(re.is_b4);
        }
        b4r = b4_policy_replay(L, state, li, rm_cols, rm_b4, add_cols, add_scores);
        if (b4r.nomem_at >= 0) {
            add_cols.resize((size_t)b4r.nomem_at + 1);
            add_scores.resize((size_t)b4r.nomem_at + 1);
        }
    }
    // out_degree as the reference keeps it
    const int64_t n_edit = (int64_t)(to_remove.size() + add_cols.size());
    if (n_edit > 0) {
        ensure_out_deg(L, true);
        if (n_edit <= DEG_INLINE) {
            DegEdits d{};
            d.n = (uint32_t)n_edit;
            uint32_t k = 0;
            for (const auto &re : to_remove) d.e[k++] = re.col | 0x80000000u;
            for (uint32_t c : add_cols) d.e[k++] = c;
            launch(k_deg_edit_inl, dim3(1), dim3(DEG_INLINE), 0, L.stream, L.out_deg.p, d);
        } else {
            // the edit list in pinned memory; its copy runs with the stream,
            // and the next call that writes the buffer waits for it (ensure)
            L.pin_deg.ensure((size_t)n_edit * 8);
            int32_t *ecol = reinterpret_cast<int32_t *>(L.pin_deg.h), *edelta = ecol + n_edit;
            int64_t k = 0;
            for (const auto &re : to_remove) {
                ecol[k] = (int32_t)re.col;
                edelta[k++] = -1;
            }
            for (uint32_t c : add_cols) {
                ecol[k] = (int32_t)c;
                edelta[k++] = 1;
            }
            TmpBuf<int32_t> dedit(L, SILI_TMPKEY(dedit));
            dedit.ensure((size_t)n_edit * 2);
            SILI_HIP(hipMemcpyAsync(dedit.p, ecol, (size_t)n_edit * 8, hipMemcpyHostToDevice, L.stream));
            L.pin_deg.mark(L.stream);
            launch(k_deg_edit, dim3(nblk(n_edit)), dim3(TPB), 0, L.stream, L.out_deg.p, (const int32_t *)dedit.p,
                   (const int32_t *)(dedit.p + n_edit), n_edit);
        }
        SILI_HIP(hipGetLastError());
    }
    if (!prune_keys.empty() || !add_cols.empty()) {
        // the device edit: explicit removals, then the inserts (weight 0,
        // importance = the probe score, delta_csr_memory.hpp:1234), as a row
        // patch of the block row, or through the bulk pipeline
        bool done = false;
        if (patch_mode) {
            BlockRowState nu = bulk_edit(L, state, prune_keys, li, add_cols, add_scores,
                                         b4r.nomem_at >= 0 ? (int64_t)b4r.nomem_bc : -1);
            for (const auto &kv : b4r.dropped) nu.tiles[kv.first] = kv.second;
            if (defer) {
                // kept on the host until an entry point other than the policy's
                // runs (policy_flush)
                auto p = L.policy_pending.find(br);
                if (p != L.policy_pending.end()) {
                    p->second.cur = std::move(nu);
                } else {
                    auto c = L.policy_clean.find(br);
                    PendingBlock pb{std::move(c->second), std::move(nu)};
                    L.policy_clean.erase(c);
                    L.policy_pending.emplace(br, std::move(pb));
                }
                done = true;
            } else {
                done = patch_block_row(L, state, nu, SB.w, SB.has_b4 ? &SB.b : nullptr);
                L.policy_clean.clear();
            }
        }
        if (!done) {
            std::vector<int32_t> cr(add_cols.size(), (int32_t)row), cc(add_cols.begin(), add_cols.end());
            std::vector<float> cv(add_cols.size(), 0.0f);
            const bool tracked = L.out_deg_tracked;
            synapto_apply(L, 0.0f, true, prune_keys.data(), (int64_t)prune_keys.size(), cr.data(), cc.data(),
                          cv.data(), add_scores.data(), (int64_t)add_cols.size(), 0, nullptr);
            L.out_deg_tracked = tracked;
            L.policy_clean.clear();
        }
    }
    if (b4r.nomem_at >= 0) {
        cursor = cursor0;
        throw_error(SILI_ERR_NOMEM, b4r.nomem_msg);
    }
    if (!no_room.empty()) {
        cursor = cursor0;
        throw_error(SILI_ERR_RUNTIME, no_room);
    }
    return true;
}

void policy_flush(Layer &L) {
    if (L.policy_pending.empty()) return;
    std::vector<const PendingBlock *> v;
    for (const auto &kv : L.policy_pending) v.push_back(&kv.second);
    bool done = false;
    if (v.size() == 1)
        done = patch_block_row(L, v[0]->orig.state, v[0]->cur, v[0]->orig.w, v[0]->orig.has_b4 ? &v[0]->orig.b : nullptr);
    if (!done) patch_blocks_rebuild_shadows(L, v);
    L.policy_pending.clear();
    L.policy_clean.clear();
}

void get_out_degree(Layer &L, int32_t *out) {
    if (L.n_out == 0) return;
    ensure_out_deg(L, false);
    SILI_HIP(hipMemcpyAsync(out, L.out_deg.p, (size_t)L.n_out * 4, hipMemcpyDeviceToHost, L.stream));
    SILI_HIP(hipStreamSynchronize(L.stream));
}

}  // namespace sili
