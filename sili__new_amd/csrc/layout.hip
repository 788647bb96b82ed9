// layout.hip -- the reference's scattered-store reservations (DeltaCSRLayout,
// delta_csr_types.hpp:763-797) kept beside the device store.
//
// The device store is compact: every structural change rebuilds it by a scan
// and a compaction, so it never needs blank space between rows.  The
// reference's store reserves, per row, index bytes and value elements beyond
// what the row holds; that reservation decides when its in-place inserts run
// out of room (synap_row_step raises) and when its budget refuses growth
// (MemoryError).  Both are part of the behaviour a caller sees, so the layer
// keeps the reference's reservation of every row (lay_b, lay_e) and applies
// the reference's rules to it:
//
//   delta_csr_from_absolute (delta_csr_memory.hpp:16-93): row r of n synapses
//     in b index bytes reserves b + floor(b * f) + 5 bytes and
//     n + max(1, floor(n * f) + 1) elements (f = blank_fraction, fp32);
//   compact (sisldo_ops.hpp:44-96): the reservation becomes the content;
//   expand_headroom[_to] (sisldo_ops.hpp:127-186): from_absolute again, after
//     the budget check its reserve() calls make;
//   delta_csr_shift_row / _equalize_step (delta_csr_memory.hpp:224-306) and
//     equalize_to_capacity (sili/cpu_backend.cpp:684-729): per-row targets,
//     the last row excepted, each growth checked against the budget.
//
// A row's content (its bytes and synapses) is read from the device store;
// the reservations live on the host (two words per row).
#include "../../include/sili_hip.h"
#include "layer.hpp"

#include <algorithm>
#include <vector>

namespace sili {

namespace {

constexpr uint64_t ULEB_MAX = 5;  // uleb128_max_bytes<uint32_t>()

// The reference's blank space for a row of `bytes` index bytes and `n`
// synapses (delta_csr_memory.hpp:59-66): size_t * float is evaluated in fp32.
inline uint64_t blank_bytes(uint64_t bytes, float f) { return (uint64_t)((float)bytes * f) + ULEB_MAX; }
inline uint64_t blank_elems(uint64_t n, float f) { return std::max<uint64_t>(1, (uint64_t)((float)n * f) + 1); }

uint64_t total(const std::vector<uint64_t> &v) {
    uint64_t s = 0;
    for (uint64_t x : v) s += x;
    return s;
}

// compact() and expand_headroom[_to] re-encode every scattered value through
// ValueAccessor<FP4BiPacked>::set(get_w, get_imp) (sisldo_ops.hpp:81-84, and
// the to_absolute / from_absolute pair): a code decodes to its table value and
// encodes back to itself, except code 8, whose NaN encodes to 0 -- in either
// nibble of the value byte (w << 4) | imp.
__global__ void k_requant_code8(uint8_t *__restrict__ val, int64_t n, int *__restrict__ changed) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const uint8_t v = val[i];
    uint8_t o = v;
    if ((v >> 4) == 8u) o &= 0x0Fu;
    if ((v & 0xFu) == 8u) o &= 0xF0u;
    if (o != v) {
        val[i] = o;
        *changed = 1;
    }
}

[[noreturn]] void out_of_budget(const char *what) {
    throw_error(SILI_ERR_NOMEM, std::string(what) + ": the layer's memory budget (set by max_weights) is exhausted");
}

// delta_csr_shift_row's bookkeeping: the byte side, then the element side,
// each only when the row is not the last; growth beyond the budget throws
// (after the byte side has moved, as in the reference).
void shift_row(Layer &L, size_t row, uint64_t tb, uint64_t te) {
    const size_t rows = L.lay_b.size();
    if (row + 1 >= rows) return;
    if (L.lay_b[row] != tb) {
        if (tb > L.lay_b[row] && total(L.lay_b) + (tb - L.lay_b[row]) > (uint64_t)L.idx_budget)
            out_of_budget("delta_csr_shift_row");
        L.lay_b[row] = tb;
    }
    if (L.lay_e[row] != te) {
        if (te > L.lay_e[row] && total(L.lay_e) + (te - L.lay_e[row]) > (uint64_t)L.val_budget)
            out_of_budget("delta_csr_shift_row");
        L.lay_e[row] = te;
    }
}

}  // namespace

void row_content(Layer &L, std::vector<uint64_t> &bytes, std::vector<uint64_t> &elems) {
    const size_t rows = (size_t)L.n_in;
    std::vector<uint32_t> bs(rows + 1, 0), es(rows + 1, 0);
    if (rows > 0 && L.W.byte_start.p) {
        BulkRead rd(L);
        rd.add(bs.data(), L.W.byte_start.p, (rows + 1) * 4);
        rd.add(es.data(), L.W.elem_start.p, (rows + 1) * 4);
        rd.wait();
    }
    bytes.resize(rows);
    elems.resize(rows);
    for (size_t r = 0; r < rows; ++r) {
        bytes[r] = bs[r + 1] - bs[r];
        elems[r] = es[r + 1] - es[r];
    }
}

void requantize_code8(Layer &L) {
    if (L.W.nnz == 0) return;
    L.scratch.flag.ensure(4, 0);
    SILI_HIP(hipMemsetAsync(L.scratch.flag.p, 0, sizeof(int), L.stream));
    const unsigned grid = (unsigned)((L.W.nnz + 255) / 256);
    for (DScatter *sc : {&L.W, &L.Wt})
        launch(k_requant_code8, dim3(grid), dim3(256), 0, L.stream, sc->val.p, sc->nnz, L.scratch.flag.p);
    SILI_HIP(hipGetLastError());
    int h = 0;
    SILI_HIP(hipMemcpyAsync(&h, L.scratch.flag.p, sizeof(int), hipMemcpyDeviceToHost, L.stream));
    SILI_HIP(hipStreamSynchronize(L.stream));
    if (!h) return;
    // copies holding value bytes are stale: rebuilt on their next use
    for (DScatter *sc : {&L.W, &L.Wt}) {
        sc->stream1.valid = sc->streamK.valid = false;
        sc->cblk.clear();
        sc->cblk_cb = 0;
    }
    refresh_nonfinite(L);
}

void layout_from_absolute(Layer &L, float blank_fraction) {
    std::vector<uint64_t> b, e;
    row_content(L, b, e);
    L.lay_b.resize(b.size());
    L.lay_e.resize(e.size());
    for (size_t r = 0; r < b.size(); ++r) {
        L.lay_b[r] = b[r] + blank_bytes(b[r], blank_fraction);
        L.lay_e[r] = e[r] + blank_elems(e[r], blank_fraction);
    }
}

void layout_compact(Layer &L) {
    requantize_code8(L);
    row_content(L, L.lay_b, L.lay_e);
}

void layout_expand(Layer &L, float blank_fraction, int64_t min_nnz_per_row) {
    // from_absolute's reserve() calls against the layer's limits
    // (delta_csr_memory.hpp:30-32, delta_csr_types.hpp:925-938), with the
    // sizes expand_headroom / expand_headroom_to ask for (double arithmetic)
    const double n = (double)L.W.nnz;
    const double budget = min_nnz_per_row < 0 ? n : std::max(n, (double)L.n_in * (double)min_nnz_per_row);
    const double grow = 1.0 + (double)blank_fraction;
    const uint64_t index_bytes = (uint64_t)(budget * grow * (double)(ULEB_MAX + 1) + 4096.0);
    const uint64_t values = (uint64_t)(budget * grow) + 64;
    const char *what = min_nnz_per_row < 0 ? "expand_headroom" : "expand_headroom_to";
    if (values > (uint64_t)L.val_budget || index_bytes > (uint64_t)L.idx_budget) out_of_budget(what);
    requantize_code8(L);
    layout_from_absolute(L, blank_fraction);
}

void layout_equalize_to_capacity(Layer &L, int64_t target_elems, int64_t target_bytes) {
    // a negative target is a size_t beyond any budget to the reference
    // (target_bytes <= 0 selects the default, as in the reference)
    if (target_elems < 0) out_of_budget("equalize_to_capacity");
    const uint64_t te = (uint64_t)target_elems;
    const uint64_t tb = target_bytes > 0 ? (uint64_t)target_bytes : te * ULEB_MAX + 4;
    const size_t rows = L.lay_b.size();
    for (size_t r = 0; r + 1 < rows; ++r) {
        const uint64_t ub = std::max(L.lay_b[r], tb), ue = std::max(L.lay_e[r], te);
        if (ub == L.lay_b[r] && ue == L.lay_e[r]) continue;
        shift_row(L, r, ub, ue);
    }
    // the last row grows without a budget check (sili/cpu_backend.cpp:715-728)
    if (rows > 0) {
        L.lay_b[rows - 1] = std::max(L.lay_b[rows - 1], tb);
        L.lay_e[rows - 1] = std::max(L.lay_e[rows - 1], te);
    }
}

void layout_equalizer_step(Layer &L) {
    const size_t rows = L.lay_b.size();
    if (rows == 0) return;
    const size_t row = (size_t)(L.eq_cursor % (int64_t)rows);
    const uint64_t tb = (total(L.lay_b) + rows - 1) / rows, te = (total(L.lay_e) + rows - 1) / rows;
    shift_row(L, row, tb, te);
    L.eq_cursor = (int64_t)((row + 1) % rows);
}

void layout_fit(Layer &L) {
    std::vector<uint64_t> b, e;
    row_content(L, b, e);
    L.lay_b.resize(b.size(), 0);
    L.lay_e.resize(e.size(), 0);
    for (size_t r = 0; r < b.size(); ++r) {
        L.lay_b[r] = std::max(L.lay_b[r], b[r]);
        L.lay_e[r] = std::max(L.lay_e[r], e[r]);
    }
}

void export_layout(Layer &L, uint64_t *byte_start, uint64_t *byte_end, uint64_t *elem_start, uint64_t *elem_end) {
    std::vector<uint64_t> b, e;
    row_content(L, b, e);
    const size_t rows = b.size();
    uint64_t pb = 0, pe = 0;
    for (size_t r = 0; r < rows; ++r) {
        if (byte_start) byte_start[r] = pb;
        if (byte_end) byte_end[r] = pb + b[r];
        if (elem_start) elem_start[r] = pe;
        if (elem_end) elem_end[r] = pe + e[r];
        pb += L.lay_b[r];
        pe += L.lay_e[r];
    }
    if (byte_start) byte_start[rows] = pb;
    if (elem_start) elem_start[rows] = pe;
}

}  // namespace sili
