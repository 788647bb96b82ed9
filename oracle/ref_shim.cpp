// ref_shim.cpp -- a thin extern "C" wrapper around the REFERENCE's own
// header-only C++ (SimLeek/sili__new sili/lib/headers), compiled in place from
// /root/reference by oracle/Makefile into oracle/_ref/libsili_ref.so.
//
// TEST INFRASTRUCTURE ONLY.  It exists to (a) pin the CPU restatement
// (sili_oracle.cpp) against the reference's real arithmetic and structure and
// write golden vectors (tests/golden/make_golden.py), and (b) time the
// reference's own CPU path as bench.py's "reference" CPU baseline.  None of
// the reference's source is copied here: the headers are #included from
// where they lie.  The product never loads this library.
#include "linear_disldo.hpp"
#include "sisldo_ops.hpp"
#include "delta_csr_memory.hpp"

#include <cstdint>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

using S = int;
using COL = uint32_t;
using Weights = SparseLinearWeightsDelta<S, FP4BiPacked, COL>;

struct RefLayer {
    Weights w;
    int n_in = 0, n_out = 0;
    // SparseLinearLayerImpl's budgets and equalizer cursors
    // (sili/cpu_backend.cpp:371-373, 646-657); SIZE_MAX: a layer built by
    // ref_layer_new[_blank], whose limits are never set
    size_t idx_budget = SIZE_MAX, val_budget = SIZE_MAX;
    size_t eq_row = 0, b4_eq_row = 0;
};

static std::string g_last_error;

template <typename F>
static int guarded_ref(F &&f) {
    try {
        f();
        return 0;
    } catch (const std::exception &e) {
        g_last_error = e.what();
        return -1;
    }
}

static CSRInput<S, float> make_input(const int32_t *ptrs, const int32_t *idx, const float *vals,
                                     int batch, int cols) {
    // Same construction as sili/cpu_backend.cpp:540-551 (_numpy_to_csr_input).
    CSRInput<S, float> csr;
    const int nz = ptrs[batch];
    csr.rows = batch;
    csr.cols = cols;
    csr.ptrs[0] = std::make_shared<std::vector<S>>(ptrs, ptrs + batch + 1);
    csr.indices[0] = std::make_shared<std::vector<S>>(idx, idx + nz);
    csr.values[0] = std::make_shared<std::vector<float>>(vals, vals + nz);
    return csr;
}

// variant 0: SparseLinearLayerDeterministic, 1: SparseLinearLayerResyncDeterministic,
// 2: SparseLinearLayerNoScaleDeterministic (sili/cpu_backend.cpp:1007-1013).
template <typename Policy, bool Deferred>
static void ref_backward_train_t(RefLayer *L, const float *x, const float *dy, int batch, float *dx, float *acc_in,
                                 float *acc_grad, float lr, int lr_per_row_nnz, int damp, float beta2, float eps,
                                 int threads) {
    disldo_backward<S, FP4BiPacked, COL, Policy, Deferred, false>(
        x, S(batch), S(L->n_in), dy, L->w, dx, acc_in, acc_grad, lr, threads, lr_per_row_nnz != 0, damp != 0,
        beta2, eps, 0.9f, 0.0f, 2.0f, 100.0f);
}

extern "C" {

uint8_t ref_fp4_encode(float v) { return fp4_encode_bits(v); }
float ref_fp4_decode(uint8_t c) { return fp4_decode_bits(c); }
float ref_fp4_table(uint8_t c) { return FP4_TABLE[c & 0xF]; }
size_t ref_uleb_encode(uint32_t v, uint8_t *out) { return uleb128_encode<uint32_t>(v, out); }

// Layer construction mirrors SparseLinearLayerImpl's constructor and
// load_weights (sili/cpu_backend.cpp:375-447, 859-901).
void *ref_layer_new_blank(int n_in, int n_out, const int32_t *ptrs, const int32_t *idx, const float *w,
                          const float *imp, float blank_fraction);

void *ref_layer_new(int n_in, int n_out, const int32_t *ptrs, const int32_t *idx,
                    const float *w, const float *imp) {
    return ref_layer_new_blank(n_in, n_out, ptrs, idx, w, imp, 0.2f);
}

// Same, with blank_fraction of per-row headroom (delta_csr_memory.hpp:17-93):
// the synaptogenesis tests give rows room to grow.
void *ref_layer_new_blank(int n_in, int n_out, const int32_t *ptrs, const int32_t *idx, const float *w,
                          const float *imp, float blank_fraction) {
    auto *L = new RefLayer();
    L->n_in = n_in;
    L->n_out = n_out;
    std::vector<S> p(ptrs, ptrs + n_in + 1);
    const size_t nnz = size_t(p.back());
    std::vector<S> ix(idx, idx + nnz);
    std::vector<float> ww(w, w + nnz);
    std::vector<float> ii(nnz, 0.0f);
    if (imp) ii.assign(imp, imp + nnz);
    L->w.connections = delta_csr_from_absolute<S, FP4BiPacked, COL>(
        p, ix, ww, ii, size_t(n_in), size_t(n_out), nnz * 8 + 4096, nnz + 64, blank_fraction);
    L->w.block4.init(size_t(n_in), size_t(n_out));
    L->w.out_degree.assign(size_t(n_out), 0);
    for (S c : ix) ++L->w.out_degree[size_t(c)];
    L->w.recompute_stats();
    return L;
}

void ref_layer_free(void *h) { delete static_cast<RefLayer *>(h); }

int ref_layer_set_scales(void *h, const float *vs, const float *os, int rank) {
    auto *L = static_cast<RefLayer *>(h);
    if (rank < 1 || size_t(rank) > Weights::SCALE_RANK_MAX) return -1;
    L->w.scale_rank = size_t(rank);
    L->w.value_scale.assign(size_t(L->n_in) * rank, 1.0f);
    for (int r = 0; r < L->n_in; ++r)
        for (int k = 0; k < rank; ++k) L->w.set_value_scale_raw_k(size_t(r), size_t(k), vs[r * rank + k]);
    if (os) {
        L->w.output_scale.assign(size_t(L->n_out) * rank, 1.0f);
        for (int c = 0; c < L->n_out; ++c)
            for (int k = 0; k < rank; ++k) L->w.set_output_scale_raw_k(size_t(c), size_t(k), os[c * rank + k]);
    }
    return 0;
}

// sili/cpu_backend.cpp:910-921 (load_dense_codes -> block4_load_dense).
void ref_layer_load_dense_codes(void *h, const uint8_t *wc, const uint8_t *ic) {
    auto *L = static_cast<RefLayer *>(h);
    block4_load_dense<S, FP4BiPacked, COL>(L->w, wc, ic, size_t(L->n_in), size_t(L->n_out));
}

// Hand-placed tile, the way the reference's own tests build block4 fixtures
// (tests/unit/test_disldo_block4_forward.cpp:34-45).
void ref_layer_put_tile(void *h, int br, int bc, const uint8_t *tile16) {
    auto *L = static_cast<RefLayer *>(h);
    auto t = L->w.block4.get_or_create(uint32_t(br), uint32_t(bc));
    for (uint32_t lj = 0; lj < 4; ++lj)
        for (uint32_t li = 0; li < 4; ++li) t.at(li, lj) = tile16[lj * 4 + li];
}

void ref_layer_compact(void *h) {
    auto *L = static_cast<RefLayer *>(h);
    L->w.connections = compact<S, FP4BiPacked, COL>(L->w.connections);
}

// Scattered structure, compacted view: per-row byte/elem starts, the row
// streams concatenated, value bytes concatenated.  Returns total index bytes.
int64_t ref_layer_export(void *h, uint64_t *byte_start, uint64_t *elem_start, uint8_t *idx,
                         uint8_t *val) {
    auto *L = static_cast<RefLayer *>(h);
    const auto &dc = L->w.connections;
    const auto &Ly = dc.layout;
    uint64_t bc = 0, ec = 0;
    for (size_t r = 0; r < Ly.rows; ++r) {
        const size_t bl = Ly.row_byte_len(r), n = Ly.row_nnz(r);
        if (byte_start) byte_start[r] = bc;
        if (elem_start) elem_start[r] = ec;
        if (idx) std::memcpy(idx + bc, dc.indices_buf.data() + Ly.byte_start[r], bl);
        if (val) std::memcpy(val + ec, dc.values._data->data() + Ly.elem_start[r], n);
        bc += bl;
        ec += n;
    }
    if (byte_start) byte_start[Ly.rows] = bc;
    if (elem_start) elem_start[Ly.rows] = ec;
    return int64_t(bc);
}

int64_t ref_layer_nnz_scattered(void *h) {
    return int64_t(static_cast<RefLayer *>(h)->w.connections.nnz());
}

// Block4 store as a list of (br, bc, 16 unpacked slot bytes) in storage order.
int64_t ref_layer_export_tiles(void *h, int32_t *br_out, int32_t *bc_out, uint8_t *tiles) {
    auto *L = static_cast<RefLayer *>(h);
    auto &B = L->w.block4;
    int64_t k = 0;
    for (size_t br = 0; br < B.block_layout.rows; ++br) {
        auto cur = B.row_cursor(br);
        const size_t n = B.block_layout.row_nnz(br);
        for (size_t e = 0; e < n; ++e) {
            const uint32_t bc = cur.advance();
            if (br_out) br_out[k] = int32_t(br);
            if (bc_out) bc_out[k] = int32_t(bc);
            if (tiles) {
                const auto t = B.find(uint32_t(br), bc);
                for (uint32_t lj = 0; lj < 4; ++lj)
                    for (uint32_t li = 0; li < 4; ++li) tiles[16 * k + lj * 4 + li] = t.at(li, lj);
            }
            ++k;
        }
    }
    return k;
}

// The block4 store's tile encoding as the reference holds it
// (block4.hpp:1016-1031): per tile its tile_is_sparse flag and its stored
// bytes (16 dense, or the sparse pack [count][positions][values],
// block4.hpp:332-388), the row's tiles concatenated without the row's
// headroom; row_used[br] = tile_byte_end - tile_byte_start.  Returns the
// packed byte count (flags and row_used may be NULL).
int64_t ref_layer_export_tiles_packed(void *h, uint8_t *flags, uint8_t *packed, uint64_t *row_used) {
    auto *L = static_cast<RefLayer *>(h);
    auto &B = L->w.block4;
    int64_t k = 0, nb = 0;
    for (size_t br = 0; br < B.block_layout.rows; ++br) {
        const size_t n = B.block_layout.row_nnz(br);
        size_t pos = B.tile_byte_start[br];
        for (size_t e = 0; e < n; ++e) {
            const size_t elem = B.block_layout.elem_start[br] + e;
            const bool sp = B.tile_is_sparse[elem] != 0;
            const size_t len = block4_stored_tile_len(sp, &B.tile_data[pos]);
            if (flags) flags[k] = sp ? 1 : 0;
            if (packed) std::memcpy(packed + nb, &B.tile_data[pos], len);
            nb += int64_t(len);
            pos += len;
            ++k;
        }
        if (row_used) row_used[br] = B.tile_byte_end[br] - B.tile_byte_start[br];
    }
    return nb;
}
// Block4Store's reservations per block row (block4.hpp:1016-1031): the
// allocated and used block-column index bytes (block_layout byte_start /
// byte_end), tile slots (elem_start / elem_end) and tile bytes
// (tile_byte_start / tile_byte_end).  out: dropped_growth_events,
// row_merge_overflow_events, row_merge_overflow_bytes_dropped,
// max_indices_bytes, max_tile_bytes.  Any array may be NULL; returns the
// block row count.
int64_t ref_block4_reservations(void *h, uint64_t *ia, uint64_t *ea, uint64_t *ta, uint64_t *ui, uint64_t *ue,
                                uint64_t *ut, uint64_t *out) {
    auto *L = static_cast<RefLayer *>(h);
    auto &B = L->w.block4;
    const auto &Ly = B.block_layout;
    for (size_t br = 0; br < Ly.rows; ++br) {
        if (ia) ia[br] = Ly.row_alloc_bytes(br);
        if (ea) ea[br] = Ly.row_alloc_elems(br);
        if (ta) ta[br] = B.tile_byte_start[br + 1] - B.tile_byte_start[br];
        if (ui) ui[br] = Ly.row_byte_len(br);
        if (ue) ue[br] = Ly.row_nnz(br);
        if (ut) ut[br] = B.tile_byte_end[br] - B.tile_byte_start[br];
    }
    if (out) {
        out[0] = B.dropped_growth_events;
        out[1] = B.row_merge_overflow_events;
        out[2] = B.row_merge_overflow_bytes_dropped;
        out[3] = B.max_indices_bytes;
        out[4] = B.max_tile_bytes;
    }
    return int64_t(Ly.rows);
}
// Block4Store::equalize_step alone (block4.hpp:1208-1220), on its own cursor;
// 0, or -1 when it throws (bad_alloc: the budget).
int ref_block4_equalize_step(void *h) {
    auto *L = static_cast<RefLayer *>(h);
    return guarded_ref([&] { L->w.block4.equalize_step(L->b4_eq_row); });
}
// block4_expand_headroom (delta_csr_memory.hpp:767-823) under the binding's
// expand_block4_headroom / compact_block4 (sili/cpu_backend.cpp:932-943):
// 0, or -1 when it throws.
int ref_block4_expand(void *h, float blank_fraction, int min_slack_bytes) {
    auto *L = static_cast<RefLayer *>(h);
    return guarded_ref([&] {
        block4_expand_headroom<S, FP4BiPacked, COL>(L->w, blank_fraction, size_t(min_slack_bytes));
    });
}
// block4_load_dense under the binding's load_dense_codes (sili/cpu_backend.cpp:
// 910-921): 0, or -1 when it throws.
int ref_sll_load_dense_codes(void *h, const uint8_t *wc, const uint8_t *ic) {
    auto *L = static_cast<RefLayer *>(h);
    return guarded_ref([&] {
        block4_load_dense<S, FP4BiPacked, COL>(L->w, wc, ic, size_t(L->n_in), size_t(L->n_out));
    });
}
// A tile placed by Block4Store::get_or_create and a handle's slot writes
// (the reference's own tests' fixture, test_disldo_block4_forward.cpp:34-45):
// 0, or -1 when get_or_create throws.
int ref_sll_put_tile(void *h, int br, int bc, const uint8_t *tile16) {
    auto *L = static_cast<RefLayer *>(h);
    return guarded_ref([&] {
        auto t = L->w.block4.get_or_create(uint32_t(br), uint32_t(bc));
        for (uint32_t lj = 0; lj < 4; ++lj)
            for (uint32_t li = 0; li < 4; ++li) t.at(li, lj) = tile16[lj * 4 + li];
    });
}

uint32_t ref_block4_switch_point(void *h, int set) {
    auto *L = static_cast<RefLayer *>(h);
    if (set >= 0) L->w.block4.switch_point = uint32_t(set);
    return L->w.block4.switch_point;
}
uint64_t ref_block4_used_bytes(void *h) {
    return static_cast<RefLayer *>(h)->w.block4.total_tile_used_bytes();
}
uint64_t ref_block4_live(void *h) { return static_cast<RefLayer *>(h)->w.block4.live_synapses(); }

int64_t ref_layer_combined(void *h, int32_t *ptrs, int32_t *idx, float *w, float *imp) {
    auto *L = static_cast<RefLayer *>(h);
    std::vector<S> op, oi;
    std::vector<float> ow, oimp;
    delta_csr_combined_to_absolute<S, FP4BiPacked, COL>(L->w, op, oi, ow, oimp);
    if (ptrs) std::memcpy(ptrs, op.data(), op.size() * sizeof(S));
    if (idx) std::memcpy(idx, oi.data(), oi.size() * sizeof(S));
    if (w) std::memcpy(w, ow.data(), ow.size() * sizeof(float));
    if (imp) std::memcpy(imp, oimp.data(), oimp.size() * sizeof(float));
    return int64_t(oi.size());
}

// sili/cpu_backend.cpp:475-492 (forward_dense): output zeroed, then accumulated.
void ref_forward_dense(void *h, const float *x, int batch, float *y, int threads) {
    auto *L = static_cast<RefLayer *>(h);
    std::memset(y, 0, sizeof(float) * size_t(batch) * size_t(L->n_out));
    disldo_forward<S, FP4BiPacked, COL>(x, S(batch), S(L->n_in), L->w, y, threads);
}

// sili/cpu_backend.cpp:496-529 (backward_dense) at learning_rate = 0 with the
// production policy constants.
void ref_backward_dense(void *h, const float *x, const float *dy, int batch, float *dx,
                        float *acc_in, float *acc_grad, int threads) {
    auto *L = static_cast<RefLayer *>(h);
    std::memset(dx, 0, sizeof(float) * size_t(batch) * size_t(L->n_in));
    disldo_backward<S, FP4BiPacked, COL>(x, S(batch), S(L->n_in), dy, L->w, dx, acc_in, acc_grad,
                                        0.0f, threads, false, true, 0.999f, 1e-8f, 0.9f, 0.0f,
                                        2.0f, 100.0f);
}

// sili/cpu_backend.cpp:496-529 (backward_dense) with the optimizer update, as
// SparseLinearLayerDeterministic runs it (sili/cpu_backend.cpp:1007:
// RMSpropScalePolicy, no deferred scale write, deterministic rounding), with
// the production policy constants.
void ref_backward_train(void *h, const float *x, const float *dy, int batch, float *dx, float *acc_in,
                        float *acc_grad, float lr, int lr_per_row_nnz, int damp, float beta2, float eps,
                        int threads, int variant) {
    auto *L = static_cast<RefLayer *>(h);
    std::memset(dx, 0, sizeof(float) * size_t(batch) * size_t(L->n_in));
    if (variant == 1)
        ref_backward_train_t<RMSpropScalePolicy<float>, true>(L, x, dy, batch, dx, acc_in, acc_grad, lr,
                                                              lr_per_row_nnz, damp, beta2, eps, threads);
    else if (variant == 2)
        ref_backward_train_t<NoScalePolicy<float>, false>(L, x, dy, batch, dx, acc_in, acc_grad, lr, lr_per_row_nnz,
                                                          damp, beta2, eps, threads);
    else
        ref_backward_train_t<RMSpropScalePolicy<float>, false>(L, x, dy, batch, dx, acc_in, acc_grad, lr,
                                                               lr_per_row_nnz, damp, beta2, eps, threads);
}

// disldo_backward_sparse_grad with the optimizer update (sili/cpu_backend.cpp:587-603).
void ref_backward_sparse_train(void *h, const float *x, const int32_t *dptrs, const int32_t *didx,
                               const float *dvals, int batch, float *dx, float *acc_in, float *acc_grad, float lr,
                               int lr_per_row_nnz, int damp, float beta2, float eps, int threads) {
    auto *L = static_cast<RefLayer *>(h);
    auto g = make_input(dptrs, didx, dvals, batch, L->n_out);
    std::memset(dx, 0, sizeof(float) * size_t(batch) * size_t(L->n_in));
    disldo_backward_sparse_grad<S, FP4BiPacked, COL>(x, S(batch), L->w, g, dx, acc_in, acc_grad, lr, threads,
                                                     lr_per_row_nnz != 0, damp != 0, beta2, eps);
}

// fp4_seed_stochastic_rng (fp4quant.hpp:186-188) on the calling thread.
void ref_seed_stochastic(uint64_t seed) { fp4_seed_stochastic_rng(seed); }

// delta_csr_build_probes (sili/cpu_backend.cpp:606-609), with the layer's
// accumulators passed in.
void ref_build_probes(void *h, const float *acc_in, const float *acc_grad, int k, int per_row) {
    auto *L = static_cast<RefLayer *>(h);
    delta_csr_build_probes<S, FP4BiPacked, COL>(L->w, acc_in, acc_grad, S(k), per_row != 0);
}

// The probe list: returns its count (the COO count), writes up to cap entries;
// *has_probes: the index vectors are non-empty.
int64_t ref_get_probes(void *h, int32_t *prow, int32_t *pcol, float *pval, int64_t cap, int *has_probes) {
    auto *L = static_cast<RefLayer *>(h);
    const auto &pr = L->w.probes;
    *has_probes = (pr.indices[0] && !pr.indices[0]->empty()) ? 1 : 0;
    const int64_t n = int64_t(pr.nnz());
    for (int64_t i = 0; i < n && i < cap; ++i) {
        prow[i] = int32_t((*pr.indices[0])[size_t(i)]);
        pcol[i] = int32_t((*pr.indices[1])[size_t(i)]);
        pval[i] = (*pr.values[0])[size_t(i)];
    }
    return n;
}

// delta_csr_synap_row_step (sili/cpu_backend.cpp:610-615): *row in/out (the
// reference advances it); returns 1/0 as it returns true/false, -2 when it
// throws (a row out of headroom).
int ref_synap_row_step(void *h, int64_t *row, float cutoff, int max_rw, int max_prune, float eps) {
    auto *L = static_cast<RefLayer *>(h);
    size_t r = size_t(*row);
    try {
        const bool did = delta_csr_synap_row_step<S, FP4BiPacked, COL>(L->w, r, cutoff, S(max_rw), S(max_prune), eps);
        *row = int64_t(r);
        return did ? 1 : 0;
    } catch (const std::exception &e) {
        g_last_error = e.what();
        *row = int64_t(r);
        return -2;
    }
}

void ref_get_out_degree(void *h, int32_t *out) {
    auto *L = static_cast<RefLayer *>(h);
    for (int c = 0; c < L->n_out; ++c) out[c] = c < int(L->w.out_degree.size()) ? int32_t(L->w.out_degree[size_t(c)]) : 0;
}

// Reserved tile bytes per block row (delta_csr_memory.hpp:767-835): with
// min_slack_bytes of room, a row's tiles can all turn dense without the
// update's eviction rule (block4.hpp merge_row_workspace) firing.
void ref_layer_block4_headroom(void *h, float blank_fraction, int min_slack_bytes) {
    auto *L = static_cast<RefLayer *>(h);
    block4_expand_headroom<S, FP4BiPacked, COL>(L->w, blank_fraction, size_t(min_slack_bytes));
}

// Per-row / per-column importance scales (delta_csr_types.hpp:1006-1031).
void ref_layer_set_importance_scales(void *h, const float *is, const float *ois) {
    auto *L = static_cast<RefLayer *>(h);
    if (is)
        for (int r = 0; r < L->n_in; ++r) L->w.set_importance_scale_raw(size_t(r), is[r]);
    if (ois)
        for (int c = 0; c < L->n_out; ++c) L->w.set_output_importance_scale_raw(size_t(c), ois[c]);
}

// The scales' optimizer state (delta_csr_types.hpp:1127-1215), rank-major
// per row / column like the scales; any pointer may be NULL.
void ref_layer_set_train_state(void *h, const float *vs_imp, const float *vs_mom, const uint32_t *vs_step,
                               const float *os_imp, const uint32_t *os_step, int os_trainable) {
    auto *L = static_cast<RefLayer *>(h);
    const size_t nr = size_t(L->n_in) * L->w.scale_rank, nc = size_t(L->n_out) * L->w.scale_rank;
    if (vs_imp) L->w.value_scale_importance.assign(vs_imp, vs_imp + nr);
    if (vs_mom) L->w.value_scale_momentum.assign(vs_mom, vs_mom + nr);
    if (vs_step) L->w.value_scale_step.assign(vs_step, vs_step + nr);
    if (os_imp) L->w.output_scale_importance.assign(os_imp, os_imp + nc);
    if (os_step) L->w.output_scale_step.assign(os_step, os_step + nc);
    if (os_trainable >= 0) L->w.output_scale_is_trainable = os_trainable != 0;
}

void ref_layer_get_train_state(void *h, float *vs, float *vs_imp, float *vs_mom, uint32_t *vs_step, float *os,
                               float *os_imp, uint32_t *os_step) {
    auto *L = static_cast<RefLayer *>(h);
    const size_t rk = L->w.scale_rank;
    for (int r = 0; r < L->n_in; ++r)
        for (size_t k = 0; k < rk; ++k) {
            const size_t i = size_t(r) * rk + k;
            if (vs) vs[i] = L->w.get_value_scale_k(size_t(r), k);
            if (vs_imp) vs_imp[i] = i < L->w.value_scale_importance.size() ? L->w.value_scale_importance[i] : 0.0f;
            if (vs_mom) vs_mom[i] = i < L->w.value_scale_momentum.size() ? L->w.value_scale_momentum[i] : 0.0f;
            if (vs_step) vs_step[i] = i < L->w.value_scale_step.size() ? L->w.value_scale_step[i] : 0u;
        }
    for (int c = 0; c < L->n_out; ++c)
        for (size_t k = 0; k < rk; ++k) {
            const size_t i = size_t(c) * rk + k;
            if (os) os[i] = L->w.get_output_scale_k(size_t(c), k);
            if (os_imp) os_imp[i] = L->w.get_output_scale_importance_k(size_t(c), k);
            if (os_step) os_step[i] = i < L->w.output_scale_step.size() ? L->w.output_scale_step[i] : 0u;
        }
}

// sili/cpu_backend.cpp:571-585 (forward_sparse).
void ref_forward_sparse(void *h, const int32_t *ptrs, const int32_t *idx, const float *vals,
                        int batch, float *y, int threads) {
    auto *L = static_cast<RefLayer *>(h);
    auto in = make_input(ptrs, idx, vals, batch, L->n_in);
    std::memset(y, 0, sizeof(float) * size_t(batch) * size_t(L->n_out));
    sisldo_forward<S, FP4BiPacked, COL>(in, L->w, y, threads);
}

// sili/cpu_backend.cpp:587-603 (backward_sparse) at learning_rate = 0.
void ref_backward_sparse(void *h, const float *x, const int32_t *dptrs, const int32_t *didx,
                         const float *dvals, int batch, float *dx, float *acc_in,
                         float *acc_grad, int threads) {
    auto *L = static_cast<RefLayer *>(h);
    auto g = make_input(dptrs, didx, dvals, batch, L->n_out);
    std::memset(dx, 0, sizeof(float) * size_t(batch) * size_t(L->n_in));
    disldo_backward_sparse_grad<S, FP4BiPacked, COL>(x, S(batch), L->w, g, dx, acc_in, acc_grad,
                                                    0.0f, threads, false, true, 0.999f, 1e-8f);
}

// Structural edits used by the synaptogenesis rules.
int ref_row_remove_col(void *h, int row, int col) {
    auto *L = static_cast<RefLayer *>(h);
    return delta_csr_row_remove_col<S, FP4BiPacked, COL>(L->w.connections, size_t(row), COL(col)) ? 1 : 0;
}
int ref_row_insert_col(void *h, int row, int col, float w, float imp) {
    auto *L = static_cast<RefLayer *>(h);
    return delta_csr_row_insert_col<S, FP4BiPacked, COL>(L->w.connections, size_t(row), COL(col), w, imp) ? 1 : 0;
}
void ref_maybe_promote(void *h, int row, int col) {
    auto *L = static_cast<RefLayer *>(h);
    block4_maybe_promote<S, FP4BiPacked, COL>(L->w, size_t(row), COL(col));
}
void ref_demote_tile(void *h, int br, int bc) {
    auto *L = static_cast<RefLayer *>(h);
    block4_demote_tile<S, FP4BiPacked, COL>(L->w, uint32_t(br), uint32_t(bc));
}
// Zero one block4 slot (the prune half of delta_csr_memory.hpp:1203-1225);
// returns the tile's live count afterwards, or -1 when the tile is absent.
int ref_zero_tile_slot(void *h, int row, int col) {
    auto *L = static_cast<RefLayer *>(h);
    auto t = L->w.block4.find(uint32_t(row / 4), uint32_t(col / 4));
    if (!t) return -1;
    t.at(uint32_t(row % 4), uint32_t(col % 4)) = 0;
    return int(t.count_live());
}

// The module's top-k conversion (csr.hpp:467-505, bound as dense_to_top_k_csr
// at sili/cpu_backend.cpp:3118-3150): returns the entry count; ptrs [rows+1],
// idx/vals sized for min(k, rows*cols).
int64_t ref_top_k_csr(float *x, int rows, int cols, int k, int threads, int32_t *ptrs, int32_t *idx, float *vals) {
    auto csr = top_k_csr<int, float>(x, size_t(rows), size_t(cols), size_t(k), threads);
    const auto &p = *csr.ptrs[0];
    const auto &i = *csr.indices[0];
    const auto &v = *csr.values[0];
    std::copy(p.begin(), p.end(), ptrs);
    std::copy(i.begin(), i.end(), idx);
    std::copy(v.begin(), v.end(), vals);
    return int64_t(i.size());
}

// ---- SparseLinearLayerImpl's reservation calls ------------------------------
// The class's own wrapper logic (sili/cpu_backend.cpp, which needs pybind and
// is not built here) restated around the header functions it calls: the
// constructor's empty layer and limits (:375-447), load_weights (:859-901),
// compact / expand_headroom[_to] (:737-790), equalize_to_capacity (:684-729)
// and equalizer_step (:646-657).  Each returns 0, or -1 when the reference
// throws (bad_alloc: the budget) with the message in ref_last_error().
const char *ref_last_error() { return g_last_error.c_str(); }

void *ref_sll_new(int n_in, int n_out, int max_weights) {
    auto *L = new RefLayer();
    L->n_in = n_in;
    L->n_out = n_out;
    L->idx_budget = size_t(max_weights) * 8 + 4096;
    L->val_budget = size_t(max_weights) + 64;
    std::vector<S> p(size_t(n_in) + 1, 0), ix;
    std::vector<float> ww, ii;
    L->w.connections = delta_csr_from_absolute<S, FP4BiPacked, COL>(p, ix, ww, ii, size_t(n_in), size_t(n_out),
                                                                    L->idx_budget, L->val_budget);
    L->w.connections.set_limits(L->idx_budget, ValueAccessor<FP4BiPacked>::projected_byte_size(L->val_budget));
    L->w.block4.init(size_t(n_in), size_t(n_out));
    L->w.block4.set_limits(size_t(max_weights) * 8 + 4096,
                           std::max<size_t>(4, size_t(max_weights) / BLOCK4_TILE_SLOTS) * BLOCK4_TILE_SLOTS);
    L->w.out_degree.assign(size_t(n_out), 0);
    L->w.recompute_stats();
    return L;
}

int ref_sll_load_weights(void *h, const int32_t *ptrs, const int32_t *idx, const float *w, const float *imp) {
    auto *L = static_cast<RefLayer *>(h);
    return guarded_ref([&] {
        std::vector<S> p(ptrs, ptrs + L->n_in + 1);
        const size_t nnz = size_t(p.back());
        std::vector<S> ix(idx, idx + nnz);
        std::vector<float> ww(w, w + nnz), ii(nnz, 0.0f);
        if (imp) ii.assign(imp, imp + nnz);
        L->idx_budget = std::max(L->idx_budget, nnz * 8 + 4096);
        L->val_budget = std::max(L->val_budget, nnz + 64);
        L->w.connections = delta_csr_from_absolute<S, FP4BiPacked, COL>(p, ix, ww, ii, size_t(L->n_in),
                                                                        size_t(L->n_out), L->idx_budget, L->val_budget);
        L->w.connections.set_limits(L->idx_budget, ValueAccessor<FP4BiPacked>::projected_byte_size(L->val_budget));
        L->w.recompute_stats();
        L->w.out_degree.assign(size_t(L->n_out), 0);
        for (S c : ix) ++L->w.out_degree[size_t(c)];
    });
}

static void reapply_limits(RefLayer *L) {
    L->w.connections.set_limits(L->idx_budget, ValueAccessor<FP4BiPacked>::projected_byte_size(L->val_budget));
}

int ref_sll_compact(void *h) {
    auto *L = static_cast<RefLayer *>(h);
    return guarded_ref([&] {
        L->w.connections = compact<S, FP4BiPacked, COL>(L->w.connections);
        reapply_limits(L);
    });
}

int ref_sll_expand(void *h, float blank_fraction) {
    auto *L = static_cast<RefLayer *>(h);
    return guarded_ref([&] {
        L->w.connections = expand_headroom<S, FP4BiPacked, COL>(L->w.connections, blank_fraction);
        reapply_limits(L);
    });
}

int ref_sll_expand_to(void *h, int min_nnz_per_row, float blank_fraction) {
    auto *L = static_cast<RefLayer *>(h);
    return guarded_ref([&] {
        L->w.connections =
            expand_headroom_to<S, FP4BiPacked, COL>(L->w.connections, size_t(min_nnz_per_row), blank_fraction);
        reapply_limits(L);
    });
}

int ref_sll_equalize_to_capacity(void *h, int target_elems, int target_bytes) {
    auto *L = static_cast<RefLayer *>(h);
    return guarded_ref([&] {
        const size_t te = size_t(target_elems);
        const size_t tb = target_bytes > 0 ? size_t(target_bytes) : te * uleb128_max_bytes<COL>() + 4;
        auto &dc = L->w.connections;
        const size_t rows = dc.layout.rows;
        for (size_t r = 0; r + 1 < rows; ++r) {
            const size_t cb = dc.layout.row_alloc_bytes(r), ce = dc.layout.row_alloc_elems(r);
            const size_t ub = std::max(cb, tb), ue = std::max(ce, te);
            if (ub == cb && ue == ce) continue;
            delta_csr_shift_row<S, FP4BiPacked, COL>(dc, r, ub, ue);
        }
        if (rows > 0) {
            auto &Ly = dc.layout;
            const size_t r = rows - 1;
            const size_t cb = Ly.row_alloc_bytes(r), ce = Ly.row_alloc_elems(r);
            const size_t ub = std::max(cb, tb), ue = std::max(ce, te);
            if (ub > cb) {
                dc.indices_buf.resize(dc.indices_buf.size() + (ub - cb), uint8_t(0));
                Ly.byte_start[rows] = Ly.byte_start[r] + ub;
            }
            if (ue > ce) {
                const size_t nt = Ly.elem_start[rows] + (ue - ce);
                ValueAccessor<FP4BiPacked>::resize(dc.values, nt);
                Ly.elem_start[rows] = nt;
            }
        }
    });
}

int ref_sll_equalizer_step(void *h) {
    auto *L = static_cast<RefLayer *>(h);
    return guarded_ref([&] {
        delta_csr_equalize_step<S, FP4BiPacked, COL>(L->w.connections, L->eq_row);
        L->w.block4.equalize_step(L->b4_eq_row);
    });
}

// The scattered layout: byte_start/elem_start [n_in+1], byte_end/elem_end [n_in].
void ref_layer_layout(void *h, uint64_t *bs, uint64_t *be, uint64_t *es, uint64_t *ee) {
    auto *L = static_cast<RefLayer *>(h);
    const auto &Ly = L->w.connections.layout;
    for (size_t r = 0; r <= Ly.rows; ++r) {
        bs[r] = Ly.byte_start[r];
        es[r] = Ly.elem_start[r];
        if (r < Ly.rows) {
            be[r] = Ly.byte_end[r];
            ee[r] = Ly.elem_end[r];
        }
    }
}

}  // extern "C"
