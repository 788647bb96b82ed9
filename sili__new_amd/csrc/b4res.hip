// b4res.hip -- the reference's block4 reservations (Block4Store,
// block4.hpp:1016-1031) kept beside the device store.
//
// The device keeps its block4 tiles dense and compact, rebuilt on every
// structural change.  The reference's store reserves, per block row, more
// block-column index bytes, tile slots and tile bytes than the row holds;
// those reservations decide when a new tile grows its row (and when the
// budget refuses that with MemoryError), when a tile's growth is dropped at
// the budget (dropped_growth_events), how much an optimizer update may grow a
// row before its write-back evicts live slots (merge_row_workspace), and what
// Block4View.alloc_bytes reports.  So the layer keeps every block row's three
// reservations (b4_ia, b4_ea, b4_ta) and applies the reference's rules:
//
//   block4_row_insert_tile (block4.hpp:670-771): a new tile takes its
//     block-column delta change, one slot and one tile byte of its row's
//     room; without room get_or_create (:1170-1183) grows the row by
//     block4_ensure_row_headroom (:648-668): +5 index bytes, +1 tile byte,
//     +1 slot, through block4_row_shift (:497-617: targets clamped to the
//     row's use; index side, tile side, slot side in that order; growth
//     beyond a budget is a MemoryError; never on the last row) or
//     block4_grow_last_row (:619-646);
//   a tile's commit (commit_dirty_sparse_tile :1226-1290 ->
//     block4_resize_tile_in_row :906-946): growth beyond the row's room
//     takes the shortfall from the store; beyond max_tile_bytes the commit
//     is dropped and counted;
//   block4_load_dense (delta_csr_memory.hpp:841-945): new budgets, a tile at
//     every (br, bc) in row-major order, each committed, then
//     block4_expand_headroom(0.2);
//   block4_expand_headroom (:767-823): ta = used + (size_t)(used * f) +
//     slack, the product in fp32; compact_block4 is f = 0, slack 0;
//   Block4Store::equalize_step (block4.hpp:1208-1220).
//
// A block row's use -- block-column ULEB128 bytes, tiles, stored tile bytes
// (sparse-packed 1 + ceil(live/2) + live, or 16) -- is read from the device
// store; the reservations live on the host (three words per block row).
#include "../../include/sili_hip.h"
#include "layer.hpp"

#include <algorithm>
#include <vector>

namespace sili {

namespace {

constexpr unsigned TPB = 256;
inline unsigned nblk(int64_t n) { return (unsigned)((n + TPB - 1) / TPB); }
constexpr uint64_t ULEB_MAX = 5;  // uleb128_max_bytes<uint32_t>()

uint64_t total(const std::vector<uint64_t> &v) {
    uint64_t s = 0;
    for (uint64_t x : v) s += x;
    return s;
}

[[noreturn]] void out_of_budget(const char *what) {
    throw_error(SILI_ERR_NOMEM, std::string(what) + ": the block4 store's memory budget is exhausted");
}

// stored bytes per block row: its tiles' lengths by tile_is_sparse and live count
// (one wave per block row, its lanes over the row's tiles)
__global__ void k_row_tile_bytes(const uint8_t *__restrict__ tiles, const uint8_t *__restrict__ flags,
                                 const uint32_t *__restrict__ tile_start, int64_t brows,
                                 uint64_t *__restrict__ out) {
    const int64_t br = (int64_t)blockIdx.x * (TPB / 64) + (threadIdx.x >> 6);
    const uint32_t lane = threadIdx.x & 63u;
    if (br >= brows) return;  // (the whole wave)
    unsigned long long s = 0;
    for (uint32_t t = tile_start[br] + lane; t < tile_start[br + 1]; t += 64u) {
        const uint4 v = *reinterpret_cast<const uint4 *>(tiles + (size_t)t * 16u);
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
        uint32_t live = 0;
        for (int i = 0; i < 4; ++i)
            for (int b = 0; b < 4; ++b) live += ((w[i] >> (8 * b)) & 0xFFu) != 0u;
        s += tile_len(flags[t] != 0, live);
    }
    for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off, 64);
    if (lane == 0) out[br] = (uint64_t)s;
}

}  // namespace

void b4res_reset(Layer &L, uint64_t idx_budget, uint64_t tile_budget) {
    const size_t rows = (size_t)((L.n_in + 3) / 4);
    L.b4_ia.assign(rows, 0);
    L.b4_ea.assign(rows, 0);
    L.b4_ta.assign(rows, 0);
    L.b4_idx_budget = idx_budget;
    L.b4_tile_budget = tile_budget;
    L.b4_ta_stale = true;
}

B4Use b4_row_use(Layer &L) {
    const int64_t rows = (L.n_in + 3) / 4;
    B4Use u;
    u.ui.assign((size_t)rows, 0);
    u.ue.assign((size_t)rows, 0);
    u.ut.assign((size_t)rows, 0);
    if (rows == 0 || L.B4.ntiles == 0) return u;
    hipStream_t st = L.stream;
    std::vector<uint32_t> bs((size_t)rows + 1), ts((size_t)rows + 1);
    TmpBuf<uint64_t> ut(L, SILI_TMPKEY(b4res_ut));
    ut.ensure((size_t)rows);
    launch(k_row_tile_bytes, dim3((unsigned)((rows + TPB / 64 - 1) / (TPB / 64))), dim3(TPB), 0, st,
           (const uint8_t *)L.B4.tiles.p, (const uint8_t *)L.B4.sparse.p, (const uint32_t *)L.B4.tile_start.p, rows,
           ut.p);
    SILI_HIP(hipGetLastError());
    BulkRead rd(L);
    rd.add(bs.data(), L.B4.byte_start.p, bs.size() * 4);
    rd.add(ts.data(), L.B4.tile_start.p, ts.size() * 4);
    rd.add(u.ut.data(), ut.p, (size_t)rows * 8);
    rd.wait();
    for (int64_t r = 0; r < rows; ++r) {
        u.ui[(size_t)r] = bs[(size_t)r + 1] - bs[(size_t)r];
        u.ue[(size_t)r] = ts[(size_t)r + 1] - ts[(size_t)r];
    }
    return u;
}

// block4_row_shift (block4.hpp:497-617) towards the three targets, each
// clamped to the row's use; nothing on the last row
void b4res_shift(Layer &L, size_t row, uint64_t ti, uint64_t tt, uint64_t te, uint64_t ui, uint64_t ue,
                 uint64_t ut) {
    ti = std::max(ti, ui);
    tt = std::max(tt, ut);
    te = std::max(te, ue);
    if (row + 1 >= L.b4_ia.size()) return;
    if (L.b4_ia[row] != ti) {
        if (ti > L.b4_ia[row] && total(L.b4_ia) + (ti - L.b4_ia[row]) > L.b4_idx_budget)
            out_of_budget("block4_row_shift");
        L.b4_ia[row] = ti;
    }
    if (L.b4_ta[row] != tt) {
        if (tt > L.b4_ta[row] && total(L.b4_ta) + (tt - L.b4_ta[row]) > L.b4_tile_budget)
            out_of_budget("block4_row_shift");
        L.b4_ta[row] = tt;
        L.b4_ta_stale = true;
    }
    if (L.b4_ea[row] != te) L.b4_ea[row] = te;
}

namespace {

// block4_grow_last_row (block4.hpp:619-646)
void grow_last(Layer &L, uint64_t ti, uint64_t tt, uint64_t te) {
    const size_t r = L.b4_ia.size() - 1;
    if (ti > L.b4_ia[r]) {
        if (total(L.b4_ia) + (ti - L.b4_ia[r]) > L.b4_idx_budget) out_of_budget("block4_grow_last_row");
        L.b4_ia[r] = ti;
    }
    if (tt > L.b4_ta[r]) {
        if (total(L.b4_ta) + (tt - L.b4_ta[r]) > L.b4_tile_budget) out_of_budget("block4_grow_last_row");
        L.b4_ta[r] = tt;
        L.b4_ta_stale = true;
    }
    if (te > L.b4_ea[r]) L.b4_ea[r] = te;
}

}  // namespace

void b4res_insert_tile(Layer &L, size_t row, int64_t idx_delta, uint64_t ui, uint64_t ue, uint64_t ut) {
    const bool fits = !(idx_delta > 0 && (uint64_t)idx_delta > L.b4_ia[row] - ui) && ue < L.b4_ea[row] &&
                      1 <= L.b4_ta[row] - ut;
    if (fits) return;
    const uint64_t ti = L.b4_ia[row] + ULEB_MAX, tt = L.b4_ta[row] + 1, te = L.b4_ea[row] + 1;
    if (row + 1 < L.b4_ia.size()) b4res_shift(L, row, ti, tt, te, ui, ue, ut);
    else grow_last(L, ti, tt, te);
}

bool b4res_commit(Layer &L, size_t row, uint64_t old_len, uint64_t new_len, uint64_t ut) {
    if (new_len <= old_len) return true;
    const uint64_t d = new_len - old_len, room = L.b4_ta[row] - ut;
    if (d <= room) return true;
    const uint64_t shortfall = d - room;
    if (total(L.b4_ta) + shortfall > L.b4_tile_budget) {
        ++L.b4_dropped;
        return false;
    }
    L.b4_ta[row] += shortfall;
    L.b4_ta_stale = true;
    return true;
}

void b4res_expand(Layer &L, float blank_fraction, uint64_t slack, const std::vector<uint64_t> &ut) {
    std::vector<uint64_t> nta(ut.size());
    uint64_t sum = 0;
    for (size_t r = 0; r < ut.size(); ++r) {
        nta[r] = ut[r] + (uint64_t)((float)ut[r] * blank_fraction) + slack;
        sum += nta[r];
    }
    if (sum > L.b4_tile_budget) out_of_budget("block4_expand_headroom");
    L.b4_ta = std::move(nta);
    L.b4_ta_stale = true;
}

void b4res_load_dense(Layer &L, const std::vector<uint8_t> &live) {
    const int64_t brows = (L.n_in + 3) / 4, bcols = (L.n_out + 3) / 4;
    const uint64_t dense_bytes = (uint64_t)brows * (uint64_t)bcols * 16u;
    b4res_reset(L, dense_bytes, (uint64_t)((double)dense_bytes * (1.0 + (double)0.2f)) + (uint64_t)brows * 16u);
    std::vector<uint64_t> ut((size_t)brows, 0);
    for (int64_t br = 0; br < brows; ++br) {
        uint64_t ui = 0, ue = 0, u = 0;
        for (int64_t bc = 0; bc < bcols; ++bc) {
            // block-column deltas 0, 1, 1, ...: one byte each; the new tile
            // is sparse-empty (1 byte) until its handle commits
            b4res_insert_tile(L, (size_t)br, 1, ui, ue, u);
            ui += 1;
            ue += 1;
            u += 1;
            const uint32_t n = live[(size_t)(br * bcols + bc)];
            const uint64_t len = tile_len(n <= L.switch_point, n);
            if (b4res_commit(L, (size_t)br, 1, len, u)) u += len - 1;
        }
        ut[(size_t)br] = u;
    }
    b4res_expand(L, 0.2f, 16, ut);
}

void b4res_put_tiles(Layer &L, int64_t n, const uint32_t *br, const uint32_t *bc, const uint8_t *tiles) {
    const size_t rows = L.b4_ia.size();
    std::vector<uint64_t> ui(rows, 0), ue(rows, 0), ut(rows, 0);
    std::vector<uint32_t> prev(rows, 0);
    for (int64_t i = 0; i < n; ++i) {
        const size_t r = br[i];
        const int64_t d = uleb_len(bc[i] - prev[r]);
        b4res_insert_tile(L, r, d, ui[r], ue[r], ut[r]);
        ui[r] += (uint64_t)d;
        ue[r] += 1;
        ut[r] += 1;
        prev[r] = bc[i];
        uint32_t live = 0;
        for (int s = 0; s < 16; ++s) live += tiles[(size_t)i * 16 + (size_t)s] != 0;
        const uint64_t len = tile_len(live <= L.switch_point, live);
        if (!b4res_commit(L, r, 1, len, ut[r]))
            out_of_budget("load_block4_tiles");  // a tile's content would be dropped
        ut[r] += len - 1;
    }
}

void b4res_equalize_step(Layer &L) {
    const size_t rows = L.b4_ia.size();
    if (rows == 0) return;
    const size_t row = (size_t)(L.b4_eq_cursor % (int64_t)rows);
    const uint64_t ti = (total(L.b4_ia) + rows - 1) / rows, tt = (total(L.b4_ta) + rows - 1) / rows,
                   te = (total(L.b4_ea) + rows - 1) / rows;
    const B4Use u = b4_row_use(L);
    b4res_shift(L, row, ti, tt, te, u.ui[row], u.ue[row], u.ut[row]);
    L.b4_eq_cursor = (int64_t)((row + 1) % rows);
}

void b4res_fit(Layer &L) {
    const B4Use u = b4_row_use(L);
    for (size_t r = 0; r < L.b4_ia.size(); ++r) {
        L.b4_ia[r] = std::max(L.b4_ia[r], u.ui[r]);
        L.b4_ea[r] = std::max(L.b4_ea[r], u.ue[r]);
        if (u.ut[r] > L.b4_ta[r]) {
            L.b4_ta[r] = u.ut[r];
            L.b4_ta_stale = true;
        }
    }
    L.b4_idx_budget = std::max(L.b4_idx_budget, total(L.b4_ia));
    L.b4_tile_budget = std::max(L.b4_tile_budget, total(L.b4_ta));
}

const uint32_t *b4_tile_cols(Layer &L) {
    if (L.B4.rng_k == 0) ensure_col_ranges(L, L.B4, 1);
    return L.B4.rng_col.p;
}

const uint32_t *b4res_device_alloc(Layer &L, hipStream_t st) {
    const size_t rows = L.b4_ta.size();
    if (L.b4_ta_stale || !L.b4_ta_dev.p) {
        std::vector<uint32_t> h(std::max<size_t>(rows, 1), 0);
        for (size_t r = 0; r < rows; ++r) h[r] = (uint32_t)std::min<uint64_t>(L.b4_ta[r], 0xFFFFFFFFull);
        L.b4_ta_dev.ensure(h.size());
        L.pin_b4ta.ensure(h.size() * 4);
        std::memcpy(L.pin_b4ta.h, h.data(), h.size() * 4);
        SILI_HIP(hipMemcpyAsync(L.b4_ta_dev.p, L.pin_b4ta.h, h.size() * 4, hipMemcpyHostToDevice, st));
        L.pin_b4ta.mark(st);
        L.b4_ta_stale = false;
    }
    return L.b4_ta_dev.p;
}

unsigned long long *b4res_counters(Layer &L, hipStream_t st) {
    if (!L.b4_ctr.p) {
        L.b4_ctr.ensure(4);
        SILI_HIP(hipMemsetAsync(L.b4_ctr.p, 0, 4 * sizeof(unsigned long long), st));
    }
    return L.b4_ctr.p;
}

void b4res_read_counters(Layer &L, uint64_t out[3]) {
    out[0] = out[1] = out[2] = 0;
    if (!L.b4_ctr.p) return;
    unsigned long long h[4] = {};
    SILI_HIP(hipMemcpyAsync(h, L.b4_ctr.p, sizeof(h), hipMemcpyDeviceToHost, L.stream));
    SILI_HIP(hipStreamSynchronize(L.stream));
    for (int i = 0; i < 3; ++i) out[i] = h[i];
}

}  // namespace sili
