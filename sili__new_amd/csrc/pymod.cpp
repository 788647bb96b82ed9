// pymod.cpp -- pybind11 module `_sili_hip`: the reference's
// `sili._cpu.SparseLinearLayer` surface (sili/cpu_backend.cpp:1506-1743) over
// the C ABI in include/sili_hip.h.  Host code only; every compute call runs
// on the GPU through libsili_hip.so.
//
// Like the reference binding, arrays are copied in and results are fresh
// arrays (never views); calls block until the GPU work is done.
#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "sili_hip.h"

namespace py = pybind11;

namespace {

[[noreturn]] void raise(int code) {
    const std::string msg = sili_last_error();
    switch (code) {
        case SILI_ERR_INVALID: throw py::value_error(msg);
        case SILI_ERR_NOMEM: throw std::bad_alloc();
        case SILI_ERR_RANGE: throw py::index_error(msg);
        default: throw std::runtime_error(msg);
    }
}
inline void ck(int code) {
    if (code != SILI_OK) raise(code);
}

template <typename T>
using carr = py::array_t<T, py::array::c_style | py::array::forcecast>;

// Page-locked host blocks behind the arrays the module returns.  A returned
// numpy array keeps its block (a capsule hands it back to the pool when the
// array dies), so a device -> host copy lands in place by DMA, and an array
// passed back in -- a chained layer's input, the backward's dy built from an
// output -- goes to the device by DMA as well.  Blocks come in 64 KiB size
// classes; at most 1 GiB of free blocks is kept, and past 2 GiB of blocks
// held by live arrays the module returns ordinary (pageable) arrays.  The
// pool is never destroyed: the HIP runtime may be gone when the interpreter
// exits.
class PinnedPool {
   public:
    static PinnedPool &get() {
        static PinnedPool *p = new PinnedPool();
        return *p;
    }
    static size_t size_class(size_t bytes) { return (bytes + 65535) & ~size_t(65535); }
    // a block of at least `bytes`, or nullptr past the live cap
    void *take(size_t bytes) {
        const size_t c = size_class(bytes ? bytes : 4);
        {
            std::lock_guard<std::mutex> g(m_);
            // the most recently freed block of the class (its pages are warm)
            auto it = free_.upper_bound(c);
            if (it != free_.begin() && (--it)->first == c) {
                void *p = it->second;
                free_.erase(it);
                free_bytes_ -= c;
                held_bytes_ += c;
                return p;
            }
            if (held_bytes_ + c > HELD_CAP) return nullptr;
        }
        void *p = nullptr;
        if (sili_host_alloc(c, &p) != SILI_OK || !p) return nullptr;
        std::lock_guard<std::mutex> g(m_);
        blocks_[(uintptr_t)p] = c;
        held_bytes_ += c;
        return p;
    }
    // whether [p, p + bytes) lies in one block of the pool
    bool owns(const void *p, size_t bytes) {
        const uintptr_t a = (uintptr_t)p;
        std::lock_guard<std::mutex> g(m_);
        auto it = blocks_.upper_bound(a);
        if (it == blocks_.begin()) return false;
        --it;
        return a >= it->first && a + bytes <= it->first + it->second;
    }
    void give(void *p) {
        size_t c = 0;
        {
            std::lock_guard<std::mutex> g(m_);
            auto it = blocks_.find((uintptr_t)p);
            if (it == blocks_.end()) return;
            c = it->second;
            held_bytes_ -= c;
            if (free_bytes_ + c <= FREE_CAP) {
                free_.emplace(c, p);
                free_bytes_ += c;
                return;
            }
            blocks_.erase(it);
        }
        (void)sili_host_free(p);
    }

   private:
    static constexpr size_t FREE_CAP = size_t(1) << 30, HELD_CAP = size_t(2) << 30;
    std::mutex m_;
    std::multimap<size_t, void *> free_;
    std::map<uintptr_t, size_t> blocks_;
    size_t free_bytes_ = 0, held_bytes_ = 0;
};

// A float32 array of `shape` over a page-locked block (pageable when the pool
// declines); *data receives its buffer.
py::array_t<float> host_array(const std::vector<py::ssize_t> &shape, float **data) {
    size_t n = 1;
    for (py::ssize_t d : shape) n *= (size_t)d;
    void *p = PinnedPool::get().take(n * 4);
    if (!p) {
        py::array_t<float> r(shape);
        *data = r.mutable_data();
        return r;
    }
    py::capsule owner(p, [](void *q) { PinnedPool::get().give(q); });
    *data = static_cast<float *>(p);
    return py::array_t<float>(shape, static_cast<float *>(p), owner);
}

// A device buffer owned by one layer wrapper, grown on demand.
struct DBuf {
    sili_layer *L = nullptr;
    void *p = nullptr;
    size_t cap = 0;
    void *get(size_t bytes) {
        if (bytes <= cap && p) return p;
        if (p) sili_device_free(L, p);
        p = nullptr;
        cap = 0;
        ck(sili_device_alloc(L, bytes ? bytes : 4, &p));
        cap = bytes;
        return p;
    }
    void release() {
        if (p && L) sili_device_free(L, p);
        p = nullptr;
        cap = 0;
    }
};

// seed_fp4_stochastic_rng: the process-wide seed every layer takes up
// before its next update (fp4quant.hpp:186-188 seeds the calling thread's
// generator).
uint64_t g_seed = 0;
uint64_t g_seed_epoch = 0;

// sili_set_update_variant's values
constexpr int UPDATE_PLAIN_V = 0, UPDATE_RESYNC_V = 1, UPDATE_NOSCALE_V = 2;

class Layer;

// Block4View (sili/cpu_backend.cpp:43-98, bound :1428-1469): the block4
// store's counters and its switch_point, read through the layer.
class Block4View {
   public:
    explicit Block4View(sili_layer *L) : L_(L) {}
    sili_block4_stats stats() const {
        sili_block4_stats st{};
        ck(sili_block4_view(L_, &st));
        return st;
    }
    int64_t tiles() const { return stats().tiles; }
    int64_t synapses() const { return stats().synapses; }
    uint32_t get_switch_point() const { return stats().switch_point; }
    void set_switch_point(uint32_t v) { ck(sili_set_switch_point(L_, v)); }
    int64_t dropped_growth_events() const { return stats().dropped_growth_events; }
    int64_t row_merge_overflow_events() const { return stats().row_merge_overflow_events; }
    int64_t row_merge_overflow_bytes_dropped() const { return stats().row_merge_overflow_bytes_dropped; }
    int64_t used_bytes() const { return stats().used_bytes; }
    int64_t alloc_bytes() const { return stats().alloc_bytes; }

   private:
    sili_layer *L_;
};

class Layer {
   public:
    Layer(int64_t n_inputs, int64_t n_outputs, int64_t max_weights, int num_cpus, int device)
        : num_cpus_(num_cpus) {
        ck(sili_create(n_inputs, n_outputs, max_weights, device, &L_));
        n_in_ = n_inputs;
        n_out_ = n_outputs;
        for (DBuf *b : bufs()) b->L = L_;
        vs_.assign((size_t)n_in_, 1.0f);
        os_.assign((size_t)n_out_, 1.0f);
        is_.assign((size_t)n_in_, 1.0f);
        ois_.assign((size_t)n_out_, 1.0f);
    }
    ~Layer() {
        for (DBuf *b : bufs()) b->release();
        sili_destroy(L_);  // waits for the stream
        release_staged();
    }
    Layer(const Layer &) = delete;
    Layer &operator=(const Layer &) = delete;

    // before an update: take up a seed_fp4_stochastic_rng issued since the last one
    void apply_seed() {
        if (seed_epoch_ != g_seed_epoch) {
            ck(sili_seed_stochastic_rounding(L_, g_seed));
            seed_epoch_ = g_seed_epoch;
        }
    }

    int64_t n_inputs() const { return n_in_; }
    int64_t n_outputs() const { return n_out_; }
    int num_cpus() const { return num_cpus_; }

    int64_t nnz() {
        sili_info info;
        ck(sili_get_info(L_, &info));
        return info.nnz_scattered + info.live_block4;
    }

    py::dict info() {
        sili_info i;
        ck(sili_get_info(L_, &i));
        py::dict d;
        d["n_inputs"] = i.n_inputs;
        d["n_outputs"] = i.n_outputs;
        d["nnz_scattered"] = i.nnz_scattered;
        d["index_bytes"] = i.index_bytes;
        d["n_tiles"] = i.n_tiles;
        d["block_index_bytes"] = i.block_index_bytes;
        d["live_block4"] = i.live_block4;
        d["n_segments"] = i.n_segments;
        d["scale_rank"] = i.scale_rank;
        d["has_nonfinite"] = bool(i.has_nonfinite);
        d["stream_canonical"] = bool(i.stream_canonical);
        d["stream_shadow"] = bool(i.stream_shadow);
        d["split_combined"] = (int)i.split_combined;
        d["short_rows_canonical"] = i.short_rows_canonical;
        d["short_rows_shadow"] = i.short_rows_shadow;
        return d;
    }

    // ---- construction ------------------------------------------------------
    void load_weights(carr<int32_t> ptrs, carr<int32_t> indices, carr<float> vals) {
        check_ptrs(ptrs, indices.size());
        if (vals.size() != indices.size()) throw py::value_error("vals and indices differ in length");
        ck(sili_load_weights(L_, ptrs.data(), indices.data(), vals.data(), nullptr, (int64_t)indices.size()));
    }
    void load_weights_with_importance(carr<int32_t> ptrs, carr<int32_t> indices, carr<float> vals,
                                      carr<float> imp) {
        check_ptrs(ptrs, indices.size());
        if (vals.size() != indices.size() || imp.size() != indices.size())
            throw py::value_error("vals/importance and indices differ in length");
        ck(sili_load_weights(L_, ptrs.data(), indices.data(), vals.data(), imp.data(), (int64_t)indices.size()));
    }
    void load_weight_bytes(carr<int32_t> ptrs, carr<int32_t> indices, carr<uint8_t> bytes) {
        check_ptrs(ptrs, indices.size());
        if (bytes.size() != indices.size()) throw py::value_error("bytes and indices differ in length");
        ck(sili_load_weight_bytes(L_, ptrs.data(), indices.data(), bytes.data(), (int64_t)indices.size()));
    }
    void load_dense_codes(carr<uint8_t> wc, carr<uint8_t> ic) {
        if (wc.size() != n_in_ * n_out_ || ic.size() != n_in_ * n_out_)
            throw py::value_error("code arrays must hold n_inputs*n_outputs entries");
        ck(sili_load_dense_codes(L_, wc.data(), ic.data()));
    }
    void load_block4_tiles(carr<int32_t> br, carr<int32_t> bc, carr<uint8_t> tiles) {
        if (br.size() != bc.size() || tiles.size() != br.size() * 16)
            throw py::value_error("need br[n], bc[n], tiles[16*n]");
        ck(sili_load_block4_tiles(L_, br.data(), bc.data(), tiles.data(), (int64_t)br.size()));
    }

    // ---- scales (host mirror, uploaded before the next compute call) --------
    int get_scale_rank() const { return rank_; }
    void set_scale_rank(int rank) {
        ck(sili_set_scale_rank(L_, rank));
        rank_ = rank;
        vs_.assign((size_t)(n_in_ * rank), 0.0f);
        os_.assign((size_t)(n_out_ * rank), 0.0f);
        for (int64_t r = 0; r < n_in_; ++r) vs_[(size_t)(r * rank)] = 1.0f;
        for (int64_t c = 0; c < n_out_; ++c) os_[(size_t)(c * rank)] = 1.0f;
        dirty_vs_ = dirty_os_ = false;
    }
    void set_value_scale_raw_k(int64_t row, int64_t k, float v) {
        check_index(row, n_in_, "row");
        check_index(k, rank_, "k");
        vs_[(size_t)(row * rank_ + k)] = v;
        dirty_vs_ = true;
    }
    void set_output_scale_raw_k(int64_t col, int64_t k, float v) {
        check_index(col, n_out_, "col");
        check_index(k, rank_, "k");
        os_[(size_t)(col * rank_ + k)] = v;
        dirty_os_ = true;
    }
    void set_value_scale_raw(int64_t row, float v) { set_value_scale_raw_k(row, 0, v); }
    void set_output_scale_raw(int64_t col, float v) { set_output_scale_raw_k(col, 0, v); }
    void set_importance_scale_raw(int64_t row, float v) {
        check_index(row, n_in_, "row");
        is_[(size_t)row] = v;
        dirty_is_ = true;
    }
    void set_output_importance_scale_raw(int64_t col, float v) {
        check_index(col, n_out_, "col");
        ois_[(size_t)col] = v;
        dirty_ois_ = true;
    }
    void set_value_scales(carr<float> v) {
        if (v.size() != n_in_ * rank_) throw py::value_error("need n_inputs*scale_rank values");
        std::memcpy(vs_.data(), v.data(), vs_.size() * 4);
        dirty_vs_ = true;
    }
    void set_output_scales(carr<float> v) {
        if (v.size() != n_out_ * rank_) throw py::value_error("need n_outputs*scale_rank values");
        std::memcpy(os_.data(), v.data(), os_.size() * 4);
        dirty_os_ = true;
    }
    float get_value_scale_k(int64_t row, int64_t k) const {
        check_index(row, n_in_, "row");
        check_index(k, rank_, "k");
        return vs_[(size_t)(row * rank_ + k)];
    }
    float get_output_scale_k(int64_t col, int64_t k) const {
        check_index(col, n_out_, "col");
        check_index(k, rank_, "k");
        return os_[(size_t)(col * rank_ + k)];
    }
    float get_value_scale(int64_t row) const { return get_value_scale_k(row, 0); }
    // bulk copies of the scale arrays, [n * rank] (flushed device state)
    py::array_t<float> get_value_scales() {
        flush();
        py::array_t<float> a((py::ssize_t)vs_.size());
        std::memcpy(a.mutable_data(), vs_.data(), vs_.size() * 4);
        return a;
    }
    float get_output_scale(int64_t col) const { return get_output_scale_k(col, 0); }
    float get_importance_scale(int64_t row) const {
        check_index(row, n_in_, "row");
        return is_[(size_t)row];
    }
    float get_output_importance_scale(int64_t col) const {
        check_index(col, n_out_, "col");
        return ois_[(size_t)col];
    }
    // delta_csr_types.hpp:1235-1240 (k >= 1 accumulated with fma, like the GPU)
    float get_scale(int64_t row, int64_t col) const {
        check_index(row, n_in_, "row");
        check_index(col, n_out_, "col");
        float s = vs_[(size_t)(row * rank_)] * os_[(size_t)(col * rank_)];
        for (int k = 1; k < rank_; ++k)
            s = __builtin_fmaf(vs_[(size_t)(row * rank_ + k)], os_[(size_t)(col * rank_ + k)], s);
        return s;
    }

    // ---- compute -------------------------------------------------------------
    py::array_t<float> forward_dense(carr<float> x) {
        flush();
        const int64_t B = x.ndim() == 2 ? (int64_t)x.shape(0) : 1;
        const int64_t cols = x.ndim() == 2 ? (int64_t)x.shape(1) : (int64_t)x.shape(0);
        if (x.ndim() > 2 || cols != n_in_) throw py::value_error("x must be [batch, n_inputs] or [n_inputs]");
        float *dx = (float *)last_x_.get((size_t)(B * n_in_) * 4);
        ck(sili_memcpy_h2d_ordered(L_, dx, stage(x.data(), (size_t)(B * n_in_) * 4), (size_t)(B * n_in_) * 4));
        last_batch_ = B;
        float *dy = (float *)y_.get((size_t)(B * n_out_) * 4);
        ck(sili_forward_dense(L_, dx, B, dy, nullptr));
        return fetch(dy, B, n_out_);
    }

    py::array_t<float> backward_dense(carr<float> dy, float learning_rate, bool lr_per_row_nnz,
                                      bool damp_by_importance, float beta2, float eps) {
        flush();
        if (last_batch_ == 0) throw std::runtime_error("backward_dense called before forward_dense");
        const int64_t B = last_batch_;
        if (dy.size() != B * n_out_) throw py::value_error("dy must be [batch, n_outputs] of the last forward");
        float *ddy = (float *)g_.get((size_t)(B * n_out_) * 4);
        ck(sili_memcpy_h2d_ordered(L_, ddy, stage(dy.data(), (size_t)(B * n_out_) * 4), (size_t)(B * n_out_) * 4));
        float *ddx = (float *)dx_.get((size_t)(B * n_in_) * 4);
        if (learning_rate == 0.0f) {
            ck(sili_backward_dense(L_, (const float *)last_x_.p, ddy, B, ddx, nullptr, nullptr, 0.0f, nullptr));
        } else {
            apply_seed();
            ck(sili_backward_dense_train(L_, (const float *)last_x_.p, ddy, B, ddx, learning_rate,
                                         lr_per_row_nnz ? 1 : 0, damp_by_importance ? 1 : 0, beta2, eps, nullptr));
            refresh_scale_mirrors();
        }
        return fetch(ddx, B, n_in_);
    }

    // an update moved the scales: refresh the host mirrors
    void refresh_scale_mirrors() {
        ck(sili_get_value_scale(L_, vs_.data()));
        ck(sili_get_output_scale(L_, os_.data()));
    }

    // The scales' optimizer state (delta_csr_types.hpp:1127-1215).
    float get_value_scale_importance(int64_t row) {
        check_index(row, n_in_, "row");
        std::vector<float> v((size_t)(n_in_ * rank_));
        ck(sili_get_scale_state(L_, v.data(), nullptr, nullptr, nullptr, nullptr));
        return v[(size_t)(row * rank_)];
    }
    float get_output_scale_importance(int64_t col) {
        check_index(col, n_out_, "col");
        std::vector<float> v((size_t)(n_out_ * rank_));
        ck(sili_get_scale_state(L_, nullptr, v.data(), nullptr, nullptr, nullptr));
        return v[(size_t)(col * rank_)];
    }
    // all of it, [n * rank] arrays
    py::dict get_scale_state() {
        const size_t nr = (size_t)(n_in_ * rank_), nc = (size_t)(n_out_ * rank_);
        py::array_t<float> vi((py::ssize_t)nr), vm((py::ssize_t)nr), oi((py::ssize_t)nc);
        py::array_t<uint32_t> vst((py::ssize_t)nr), ost((py::ssize_t)nc);
        ck(sili_get_scale_state(L_, vi.mutable_data(), oi.mutable_data(), vm.mutable_data(), vst.mutable_data(),
                                ost.mutable_data()));
        py::dict d;
        d["vs_importance"] = vi;
        d["vs_momentum"] = vm;
        d["vs_step"] = vst;
        d["os_importance"] = oi;
        d["os_step"] = ost;
        return d;
    }
    void seed_stochastic_rounding(uint64_t seed) {
        ck(sili_seed_stochastic_rounding(L_, seed));
        seed_epoch_ = g_seed_epoch;
    }

    // nnz-sampled grad-W for (x, dy): (per scattered synapse, per block4 slot)
    py::tuple sampled_gradw(carr<float> x, carr<float> dy) {
        flush();
        const int64_t B = x.ndim() == 2 ? (int64_t)x.shape(0) : 1;
        if (x.size() != B * n_in_ || dy.size() != B * n_out_) throw py::value_error("x [B,n_in], dy [B,n_out]");
        sili_info i;
        ck(sili_get_info(L_, &i));
        // x goes to its own buffer: the stored forward input (last_input)
        // belongs to forward_dense alone, as the reference's _last_input
        float *dx = (float *)xs_.get((size_t)(B * n_in_) * 4);
        float *dg = (float *)g_.get((size_t)(B * n_out_) * 4);
        ck(sili_memcpy_h2d_ordered(L_, dx, stage(x.data(), (size_t)(B * n_in_) * 4), (size_t)(B * n_in_) * 4));
        ck(sili_memcpy_h2d_ordered(L_, dg, stage(dy.data(), (size_t)(B * n_out_) * 4), (size_t)(B * n_out_) * 4));
        float *gs = (float *)gws_.get((size_t)i.nnz_scattered * 4 + 4);
        float *gb = (float *)gwb_.get((size_t)i.n_tiles * 64 + 4);
        ck(sili_sampled_gradw(L_, dx, dg, B, gs, gb, nullptr));
        float *ha = nullptr, *hb = nullptr;
        py::array_t<float> a = host_array({(py::ssize_t)i.nnz_scattered}, &ha);
        py::array_t<float> b = host_array({(py::ssize_t)(i.n_tiles * 16)}, &hb);
        ck(sili_memcpy_d2h_ordered(L_, ha, gs, (size_t)i.nnz_scattered * 4));
        ck(sili_memcpy_d2h_ordered(L_, hb, gb, (size_t)i.n_tiles * 64));
        release_staged();
        return py::make_tuple(a, b);
    }

    py::array_t<float> forward_sparse(carr<int32_t> ptrs, carr<int32_t> indices, carr<float> values,
                                      int64_t batch) {
        flush();
        check_csr(ptrs, indices, values, batch, n_in_);
        int32_t *dp = upload_i32(p_, ptrs);
        int32_t *di = upload_i32(i_, indices);
        float *dv = upload_f32(v_, values);
        float *dy = (float *)y_.get((size_t)(batch * n_out_) * 4);
        ck(sili_forward_sparse(L_, dp, di, dv, (int64_t)indices.size(), batch, dy, nullptr));
        return fetch(dy, batch, n_out_);
    }

    py::array_t<float> backward_sparse(carr<float> x, carr<int32_t> dptrs, carr<int32_t> didx, carr<float> dvals,
                                       int64_t batch, float learning_rate, bool lr_per_row_nnz,
                                       bool damp_by_importance, float beta2, float eps) {
        flush();
        if (x.size() != batch * n_in_) throw py::value_error("x must be [batch, n_inputs]");
        check_csr(dptrs, didx, dvals, batch, n_out_);
        float *dxin = (float *)xs_.get((size_t)(batch * n_in_) * 4);
        ck(sili_memcpy_h2d_ordered(L_, dxin, stage(x.data(), (size_t)(batch * n_in_) * 4), (size_t)(batch * n_in_) * 4));
        int32_t *dp = upload_i32(p_, dptrs);
        int32_t *di = upload_i32(i_, didx);
        float *dv = upload_f32(v_, dvals);
        float *ddx = (float *)dx_.get((size_t)(batch * n_in_) * 4);
        ck(sili_backward_sparse_train(L_, dxin, dp, di, dv, (int64_t)didx.size(), batch, ddx, learning_rate,
                                      lr_per_row_nnz ? 1 : 0, damp_by_importance ? 1 : 0, beta2, eps, nullptr));
        if (learning_rate != 0.0f) refresh_scale_mirrors();
        return fetch(ddx, batch, n_in_);
    }

    // ---- synaptogenesis ---------------------------------------------------------
    py::dict synapto_step(float prune_frac, carr<int32_t> rows, carr<int32_t> cols, carr<float> vals,
                          py::object scores, int default_imp_code) {
        flush();
        if (rows.size() != cols.size() || vals.size() != rows.size())
            throw py::value_error("candidate arrays differ in length");
        const float *sp = nullptr;
        carr<float> sarr;
        if (!scores.is_none()) {
            sarr = scores.cast<carr<float>>();
            if (sarr.size() != rows.size()) throw py::value_error("scores length differs");
            sp = sarr.data();
        }
        int64_t st[7] = {0, 0, 0, 0, 0, 0, 0};
        ck(sili_synapto_step(L_, prune_frac, rows.data(), cols.data(), vals.data(), sp, (int64_t)rows.size(),
                             default_imp_code, st));
        py::dict d;
        const char *names[7] = {"n_prune_target", "n_pruned", "n_grown", "n_demoted_tiles",
                                "n_promoted_tiles", "n_scattered", "n_tiles"};
        for (int k = 0; k < 7; ++k) d[names[k]] = st[k];
        return d;
    }

    // Seeded synthetic layer generated on the device (benchmark workloads);
    // the value-scale mirror is refreshed from the device afterwards.
    int64_t load_synthetic(uint64_t seed, double keep_prob, float sigma, float tail_q) {
        flush();
        int64_t nnz = 0;
        ck(sili_load_synthetic(L_, seed, keep_prob, sigma, tail_q, &nnz));
        ck(sili_get_value_scale(L_, vs_.data()));
        dirty_vs_ = false;
        return nnz;
    }

    // The reference's reservation management (sisldo_ops.hpp:44-186,
    // delta_csr_memory.hpp:224-306, sili/cpu_backend.cpp:649-790): the device
    // store stays compact while the layer keeps, per row, what the reference's
    // store would reserve (export_layout), so that synap_row_step runs out of
    // room and growth meets the budget where the reference's do.
    void compact() {
        flush();
        ck(sili_compact(L_));
    }
    void expand_headroom(float bf) {
        flush();
        ck(sili_expand_headroom(L_, bf));
    }
    void expand_headroom_to(int m, float bf) {
        flush();
        ck(sili_expand_headroom_to(L_, m, bf));
    }
    void equalizer_step() { ck(sili_equalizer_step(L_)); }
    void equalize_to_capacity(int te, int tb) { ck(sili_equalize_to_capacity(L_, te, tb)); }
    // the block rows' tile-byte reservations (sili/cpu_backend.cpp:932-943)
    void expand_block4_headroom(float bf) { ck(sili_expand_block4_headroom(L_, bf)); }
    void compact_block4() { ck(sili_compact_block4(L_)); }
    // the block4 store's reservations per block row, as the reference's
    // Block4Store holds them (sili_export_block4_layout)
    py::dict export_block4_layout() {
        const py::ssize_t rows = (py::ssize_t)((n_in_ + 3) / 4);
        py::array_t<uint64_t> ia(rows), ea(rows), ta(rows), ui(rows), ue(rows), ut(rows), out(6);
        ck(sili_export_block4_layout(L_, ia.mutable_data(), ea.mutable_data(), ta.mutable_data(), ui.mutable_data(),
                                     ue.mutable_data(), ut.mutable_data(), out.mutable_data()));
        py::dict d;
        d["ia"] = ia;
        d["ea"] = ea;
        d["ta"] = ta;
        d["ui"] = ui;
        d["ue"] = ue;
        d["ut"] = ut;
        auto o = out.unchecked<1>();
        d["dropped_growth_events"] = o(0);
        d["row_merge_overflow_events"] = o(1);
        d["row_merge_overflow_bytes_dropped"] = o(2);
        d["idx_budget"] = o(3);
        d["tile_budget"] = o(4);
        d["evicted"] = o(5);
        return d;
    }
    py::dict export_layout() {
        py::array_t<uint64_t> bs((py::ssize_t)(n_in_ + 1)), be((py::ssize_t)n_in_), es((py::ssize_t)(n_in_ + 1)),
            ee((py::ssize_t)n_in_);
        ck(sili_export_layout(L_, bs.mutable_data(), be.mutable_data(), es.mutable_data(), ee.mutable_data()));
        py::dict d;
        d["byte_start"] = bs;
        d["byte_end"] = be;
        d["elem_start"] = es;
        d["elem_end"] = ee;
        return d;
    }
    // test hook: digests of the internal stores (sili_debug_store_digest)
    py::array_t<uint64_t> _store_digest() {
        py::array_t<uint64_t> d(6);
        ck(sili_debug_store_digest(L_, d.mutable_data()));
        return d;
    }

    // ---- accumulators / exports -----------------------------------------------
    py::array_t<float> neuron_input_accum() {
        py::array_t<float> a((py::ssize_t)n_in_);
        ck(sili_get_accumulators(L_, a.mutable_data(), nullptr));
        return a;
    }
    py::array_t<float> neuron_grad_accum() {
        py::array_t<float> a((py::ssize_t)n_out_);
        ck(sili_get_accumulators(L_, nullptr, a.mutable_data()));
        return a;
    }
    void zero_accum() { ck(sili_zero_accum(L_)); }

    py::tuple absolute() {
        int64_t n = 0;
        ck(sili_export_absolute(L_, nullptr, nullptr, nullptr, nullptr, &n));
        py::array_t<int32_t> p((py::ssize_t)(n_in_ + 1)), ix((py::ssize_t)n);
        py::array_t<float> w((py::ssize_t)n), imp((py::ssize_t)n);
        ck(sili_export_absolute(L_, p.mutable_data(), ix.mutable_data(), w.mutable_data(), imp.mutable_data(), &n));
        return py::make_tuple(p, ix, w, imp);
    }
    py::array_t<int32_t> ptrs() { return absolute()[0].cast<py::array_t<int32_t>>(); }
    py::array_t<int32_t> indices() { return absolute()[1].cast<py::array_t<int32_t>>(); }
    py::array_t<float> weights_vals() { return absolute()[2].cast<py::array_t<float>>(); }
    py::array_t<float> importance() { return absolute()[3].cast<py::array_t<float>>(); }
    py::array_t<int32_t> out_degree() {
        py::array_t<int32_t> d((py::ssize_t)n_out_);
        if (n_out_ > 0) ck(sili_get_out_degree(L_, d.mutable_data()));
        return d;
    }

    // ---- the reference's synaptogenesis policy (sili/cpu_backend.cpp:606-634) ----
    void build_probes(int64_t k, bool per_row) {
        flush();
        ck(sili_build_probes(L_, k, per_row ? 1 : 0));
    }
    bool synap_row_step(int64_t current_row, float importance_cutoff, int64_t max_row_weights,
                        int64_t max_prune_per_step, float importance_eps) {
        flush();
        int did = 0;
        ck(sili_synap_row_step(L_, &current_row, importance_cutoff, max_row_weights, max_prune_per_step,
                               importance_eps, &did));
        return did != 0;
    }
    bool synap_step(float importance_cutoff, int64_t max_row_weights, int64_t max_prune_per_step,
                    float importance_eps) {
        flush();
        int did = 0;
        ck(sili_synap_step(L_, importance_cutoff, max_row_weights, max_prune_per_step, importance_eps, &did));
        return did != 0;
    }
    py::tuple get_probes() {
        int64_t n = 0;
        ck(sili_get_probes(L_, &n, nullptr, nullptr, nullptr, 0));
        py::array_t<int32_t> r((py::ssize_t)n), c((py::ssize_t)n);
        py::array_t<float> v((py::ssize_t)n);
        ck(sili_get_probes(L_, &n, r.mutable_data(), c.mutable_data(), v.mutable_data(), n));
        return py::make_tuple(r, c, v);
    }
    py::object last_input() {
        if (last_batch_ == 0) return py::none();
        return fetch((const float *)last_x_.p, last_batch_, n_in_);
    }

    py::dict export_scattered() {
        sili_info i;
        ck(sili_get_info(L_, &i));
        py::array_t<uint64_t> bs((py::ssize_t)(n_in_ + 1)), es((py::ssize_t)(n_in_ + 1));
        py::array_t<uint8_t> ix((py::ssize_t)i.index_bytes), v((py::ssize_t)i.nnz_scattered);
        ck(sili_export_scattered(L_, bs.mutable_data(), es.mutable_data(), ix.mutable_data(), v.mutable_data()));
        py::dict d;
        d["row_byte_start"] = bs;
        d["row_elem_start"] = es;
        d["idx"] = ix;
        d["val"] = v;
        return d;
    }
    py::dict export_block4() {
        sili_info i;
        ck(sili_get_info(L_, &i));
        const int64_t brows = (n_in_ + 3) / 4;
        py::array_t<int32_t> br((py::ssize_t)i.n_tiles), bc((py::ssize_t)i.n_tiles);
        py::array_t<uint8_t> t((py::ssize_t)(i.n_tiles * 16)), bix((py::ssize_t)i.block_index_bytes);
        py::array_t<uint64_t> bs((py::ssize_t)(brows + 1)), ts((py::ssize_t)(brows + 1));
        ck(sili_export_block4(L_, br.mutable_data(), bc.mutable_data(), t.mutable_data(), bs.mutable_data(),
                              ts.mutable_data(), bix.mutable_data()));
        py::dict d;
        d["br"] = br;
        d["bc"] = bc;
        d["tiles"] = t;
        d["brow_byte_start"] = bs;
        d["brow_tile_start"] = ts;
        d["bidx"] = bix;
        return d;
    }
    Block4View block4() { return Block4View(L_); }
    // the reference's stored tile encoding: tile_is_sparse, tile_data (rows
    // concatenated without headroom) and each block row's first byte
    py::dict export_block4_packed() {
        int64_t nb = 0;
        sili_info i;
        ck(sili_get_info(L_, &i));
        ck(sili_export_block4_packed(L_, nullptr, nullptr, nullptr, &nb));
        py::array_t<uint8_t> f((py::ssize_t)i.n_tiles), d((py::ssize_t)nb);
        py::array_t<uint64_t> rs((py::ssize_t)((n_in_ + 3) / 4 + 1));
        ck(sili_export_block4_packed(L_, f.mutable_data(), d.mutable_data(), rs.mutable_data(), &nb));
        py::dict out;
        out["tile_is_sparse"] = f;
        out["tile_data"] = d;
        out["tile_byte_start"] = rs;
        return out;
    }

    // the FOR index of the canonical store (derived copy, built on request)
    void build_for_index(int group_size) { ck(sili_build_for_index(L_, group_size)); }
    py::dict export_for_index() {
        int64_t nb = 0;
        ck(sili_export_for_index(L_, nullptr, nullptr, &nb));
        py::array_t<uint64_t> rs((py::ssize_t)(n_in_ + 1));
        py::array_t<uint8_t> b((py::ssize_t)nb);
        ck(sili_export_for_index(L_, rs.mutable_data(), b.mutable_data(), &nb));
        py::dict d;
        d["row_byte_start"] = rs;
        d["bytes"] = b;
        return d;
    }
    py::array_t<int32_t> decode_columns(int use_for_index) {
        sili_info i;
        ck(sili_get_info(L_, &i));
        py::array_t<int32_t> c((py::ssize_t)i.nnz_scattered);
        if (i.nnz_scattered == 0) return c;
        int32_t *d = (int32_t *)dx_.get((size_t)i.nnz_scattered * 4);
        ck(sili_decode_columns(L_, d, use_for_index, nullptr));
        ck(sili_memcpy_d2h(L_, c.mutable_data(), d, (size_t)i.nnz_scattered * 4));
        return c;
    }
    py::tuple decode_scattered() {
        sili_info i;
        ck(sili_get_info(L_, &i));
        flush();
        py::array_t<int32_t> c((py::ssize_t)i.nnz_scattered);
        py::array_t<float> w((py::ssize_t)i.nnz_scattered);
        ck(sili_decode_scattered(L_, c.mutable_data(), w.mutable_data()));
        return py::make_tuple(c, w);
    }
    void synchronize() { ck(sili_synchronize(L_)); }
    uintptr_t handle() const { return reinterpret_cast<uintptr_t>(L_); }
    // rounding of the update's re-quantization (stochastic by default)
    void set_stochastic_rounding(bool on) { ck(sili_set_stochastic_rounding(L_, on ? 1 : 0)); }
    // the update's scale-update variant (0 plain, 1 resync, 2 noscale)
    void set_update_variant(int v) { ck(sili_set_update_variant(L_, v)); }

   private:
    sili_layer *L_ = nullptr;
    uint64_t seed_epoch_ = 0;
    int64_t n_in_ = 0, n_out_ = 0;
    int num_cpus_ = 4;
    int rank_ = 1;
    std::vector<float> vs_, os_, is_, ois_;
    bool dirty_vs_ = false, dirty_os_ = false, dirty_is_ = false, dirty_ois_ = false;
    int64_t last_batch_ = 0;
    DBuf last_x_, xs_, y_, g_, dx_, p_, i_, v_, gws_, gwb_;
    std::vector<void *> staged_;  // pool blocks that queued uploads read

    std::vector<DBuf *> bufs() { return {&last_x_, &xs_, &y_, &g_, &dx_, &p_, &i_, &v_, &gws_, &gwb_}; }

    void flush() {
        if (dirty_vs_) ck(sili_set_value_scale(L_, vs_.data()));
        if (dirty_os_) ck(sili_set_output_scale(L_, os_.data()));
        if (dirty_is_) ck(sili_set_importance_scale(L_, is_.data()));
        if (dirty_ois_) ck(sili_set_output_importance_scale(L_, ois_.data()));
        dirty_vs_ = dirty_os_ = dirty_is_ = dirty_ois_ = false;
    }
    static void check_index(int64_t i, int64_t n, const char *what) {
        if (i < 0 || i >= n) throw py::index_error(std::string(what) + " out of range");
    }
    void check_ptrs(const carr<int32_t> &ptrs, py::ssize_t nnz) const {
        if (ptrs.size() != n_in_ + 1) throw py::value_error("ptrs must have n_inputs+1 entries");
        if (ptrs.data()[n_in_] != nnz) throw py::value_error("ptrs[-1] must equal len(indices)");
    }
    static void check_csr(const carr<int32_t> &ptrs, const carr<int32_t> &idx, const carr<float> &vals,
                          int64_t batch, int64_t n) {
        if (batch <= 0) throw py::value_error("batch must be >= 1");
        if (ptrs.size() != batch + 1) throw py::value_error("ptrs must have batch+1 entries");
        if (idx.size() != vals.size()) throw py::value_error("indices and values differ in length");
        const int32_t *p = ptrs.data();
        if (p[0] != 0 || p[batch] != (int32_t)idx.size()) throw py::value_error("ptrs must span the indices");
        for (int64_t b = 0; b < batch; ++b)
            if (p[b + 1] < p[b]) throw py::value_error("ptrs must be non-decreasing");
        const int32_t *ix = idx.data();
        for (int64_t b = 0; b < batch; ++b)
            for (int64_t k = p[b]; k < p[b + 1]; ++k) {
                if (ix[k] < 0 || ix[k] >= n) throw py::value_error("sparse index out of range");
                if (k > p[b] && ix[k] <= ix[k - 1])
                    throw py::value_error("sparse indices must be strictly increasing within a batch row");
            }
    }
    // (uploads are ordered on the layer's stream without a wait: every entry
    // point that makes them returns through fetch or an ordered device ->
    // host copy, which waits for the stream, while its arguments are alive)
    int32_t *upload_i32(DBuf &b, const carr<int32_t> &a) {
        void *d = b.get((size_t)a.size() * 4 + 4);
        ck(sili_memcpy_h2d_ordered(L_, d, stage(a.data(), (size_t)a.size() * 4), (size_t)a.size() * 4));
        return (int32_t *)d;
    }
    float *upload_f32(DBuf &b, const carr<float> &a) {
        void *d = b.get((size_t)a.size() * 4 + 4);
        ck(sili_memcpy_h2d_ordered(L_, d, stage(a.data(), (size_t)a.size() * 4), (size_t)a.size() * 4));
        return (float *)d;
    }
    py::array_t<float> fetch(const float *d, int64_t B, int64_t n) {
        float *h = nullptr;
        py::array_t<float> r = host_array({(py::ssize_t)B, (py::ssize_t)n}, &h);
        ck(sili_memcpy_d2h_ordered(L_, h, d, (size_t)(B * n) * 4));
        release_staged();
        return r;
    }
    // The host source of an upload: an array of this module's pool as it is
    // (page-locked: one copy kernel reads it), else, from 64 KiB up, a copy in
    // a page-locked block of the pool (a CPU copy of a few tens of us per
    // 2 MiB, where the runtime's staged copy of pageable memory took 0.08 ms
    // and, on streams where its DMA runs slow, 0.3 ms).  The block is held
    // until a wait for the layer's stream (release_staged).
    const void *stage(const void *src, size_t bytes) {
        if (bytes < (size_t(64) << 10) || PinnedPool::get().owns(src, bytes)) return src;
        void *p = PinnedPool::get().take(bytes);
        if (!p) return src;
        std::memcpy(p, src, bytes);
        staged_.push_back(p);
        return p;
    }
    // after a wait for the layer's stream: the staged blocks go back
    void release_staged() {
        for (void *p : staged_) PinnedPool::get().give(p);
        staged_.clear();
    }
};

// A device buffer of the module utilities (no layer): freed on scope exit.
struct UBuf {
    int dev = 0;
    void *p = nullptr;
    UBuf(int device, size_t bytes) : dev(device) { ck(sili_buffer_alloc(device, bytes, &p)); }
    ~UBuf() {
        if (p) (void)sili_buffer_free(dev, p);
    }
    UBuf(const UBuf &) = delete;
    UBuf &operator=(const UBuf &) = delete;
    void put(const void *h, size_t bytes) {
        if (bytes) ck(sili_buffer_copy(dev, p, h, bytes));
    }
    void get(void *h, size_t bytes) const {
        if (bytes) ck(sili_buffer_copy(dev, h, p, bytes));
    }
};

// fp4_quantize_array (sili/cpu_backend.cpp:3157): fp32 -> uint8 codes, on the GPU.
py::array_t<uint8_t> fp4_quantize_array(carr<float> v, int device) {
    py::array_t<uint8_t> out(v.request().shape);
    const size_t n = (size_t)v.size();
    if (n == 0) return out;
    UBuf dx(device, 4 * n), dc(device, n);
    dx.put(v.data(), 4 * n);
    ck(sili_fp4_quantize(static_cast<const float *>(dx.p), (int64_t)n, static_cast<uint8_t *>(dc.p), nullptr));
    dc.get(out.mutable_data(), n);
    return out;
}

// [batch, cols] or [cols] -> (rows, cols) as the reference binding reads them
std::pair<int64_t, int64_t> csr_shape(const carr<float> &x) {
    const auto b = x.request();
    if (b.ndim == 2) return {(int64_t)b.shape[0], (int64_t)b.shape[1]};
    if (b.ndim == 1) return {1, (int64_t)b.shape[0]};
    throw py::value_error("expected a 1-D or 2-D float32 array");
}

// dense_to_csr (sili/cpu_backend.cpp:3075-3116): entries with |v| > threshold.
py::tuple dense_to_csr(carr<float> x, float threshold, int device) {
    const auto [rows, cols] = csr_shape(x);
    const size_t n = (size_t)(rows * cols);
    UBuf dx(device, 4 * n + 4), dp(device, 4 * ((size_t)rows + 1)), di(device, 4 * n + 4), dv(device, 4 * n + 4);
    dx.put(x.data(), 4 * n);
    int64_t nnz = 0;
    ck(sili_dense_to_csr(static_cast<const float *>(dx.p), rows, cols, threshold, static_cast<int32_t *>(dp.p),
                         static_cast<int32_t *>(di.p), static_cast<float *>(dv.p), (int64_t)n, &nnz, nullptr));
    py::array_t<int32_t> ptrs((py::ssize_t)(rows + 1)), idx((py::ssize_t)nnz);
    py::array_t<float> vals((py::ssize_t)nnz);
    dp.get(ptrs.mutable_data(), 4 * ((size_t)rows + 1));
    di.get(idx.mutable_data(), 4 * (size_t)nnz);
    dv.get(vals.mutable_data(), 4 * (size_t)nnz);
    return py::make_tuple(ptrs, idx, vals);
}

// dense_to_top_k_csr (sili/cpu_backend.cpp:3118-3150): global top-k by |v|.
// num_threads is the reference's OpenMP width; the GPU ignores it.
py::tuple dense_to_top_k_csr(carr<float> x, int64_t k, int num_threads, int device) {
    (void)num_threads;
    const auto [rows, cols] = csr_shape(x);
    if (k < 0) throw py::value_error("k must be >= 0");
    const size_t n = (size_t)(rows * cols);
    const size_t kk = std::min<size_t>((size_t)k, n);
    UBuf dx(device, 4 * n + 4), dp(device, 4 * ((size_t)rows + 1)), di(device, 4 * kk + 4), dv(device, 4 * kk + 4);
    dx.put(x.data(), 4 * n);
    int64_t nnz = 0;
    ck(sili_dense_to_top_k_csr(static_cast<const float *>(dx.p), rows, cols, k, static_cast<int32_t *>(dp.p),
                               static_cast<int32_t *>(di.p), static_cast<float *>(dv.p), &nnz, nullptr));
    py::array_t<int32_t> ptrs((py::ssize_t)(rows + 1)), idx((py::ssize_t)nnz);
    py::array_t<float> vals((py::ssize_t)nnz);
    dp.get(ptrs.mutable_data(), 4 * ((size_t)rows + 1));
    di.get(idx.mutable_data(), 4 * (size_t)nnz);
    dv.get(vals.mutable_data(), 4 * (size_t)nnz);
    return py::make_tuple(ptrs, idx, vals);
}

// The reference's other concrete layer classes (sili/cpu_backend.cpp:992-1013):
// the same layer with another scale-update variant of the optimizer update
// (sili_set_update_variant) and/or round-to-nearest re-quantization.
template <int Variant, bool Stochastic>
class LayerVariant : public Layer {
   public:
    LayerVariant(int64_t n_inputs, int64_t n_outputs, int64_t max_weights, int num_cpus, int device)
        : Layer(n_inputs, n_outputs, max_weights, num_cpus, device) {
        set_stochastic_rounding(Stochastic);
        set_update_variant(Variant);
    }
};
using LayerDeterministic = LayerVariant<UPDATE_PLAIN_V, false>;
using LayerResync = LayerVariant<UPDATE_RESYNC_V, true>;
using LayerResyncDeterministic = LayerVariant<UPDATE_RESYNC_V, false>;
using LayerNoScale = LayerVariant<UPDATE_NOSCALE_V, true>;
using LayerNoScaleDeterministic = LayerVariant<UPDATE_NOSCALE_V, false>;

template <typename T>
void bind_variant(py::module_ &m, const char *name) {
    py::class_<T, Layer>(m, name)
        .def(py::init<int64_t, int64_t, int64_t, int, int>(), py::arg("n_inputs"), py::arg("n_outputs"),
             py::arg("max_weights"), py::arg("num_cpus") = 4, py::arg("device") = 0);
}

}  // namespace

PYBIND11_MODULE(_sili_hip, m) {
    m.doc() = "gfx950 FP4 delta-CSR sparse linear layer (sili SparseLinearLayer API)";
    py::class_<Block4View>(m, "Block4View")
        .def_property_readonly("tiles", &Block4View::tiles)
        .def_property_readonly("synapses", &Block4View::synapses)
        .def_property("switch_point", &Block4View::get_switch_point, &Block4View::set_switch_point)
        .def_property_readonly("dropped_growth_events", &Block4View::dropped_growth_events)
        .def_property_readonly("row_merge_overflow_events", &Block4View::row_merge_overflow_events)
        .def_property_readonly("row_merge_overflow_bytes_dropped", &Block4View::row_merge_overflow_bytes_dropped)
        .def_property_readonly("used_bytes", &Block4View::used_bytes)
        .def_property_readonly("alloc_bytes", &Block4View::alloc_bytes);
    py::class_<Layer>(m, "SparseLinearLayer")
        .def(py::init<int64_t, int64_t, int64_t, int, int>(), py::arg("n_inputs"), py::arg("n_outputs"),
             py::arg("max_weights"), py::arg("num_cpus") = 4, py::arg("device") = 0)
        .def("load_weights", &Layer::load_weights, py::arg("ptrs"), py::arg("indices"), py::arg("vals"))
        .def("load_weights_with_importance", &Layer::load_weights_with_importance)
        .def("load_weight_bytes", &Layer::load_weight_bytes)
        .def("load_dense_codes", &Layer::load_dense_codes, py::arg("weight_codes"), py::arg("importance_codes"))
        .def("load_block4_tiles", &Layer::load_block4_tiles, py::arg("br"), py::arg("bc"), py::arg("tiles"))
        .def("load_synthetic", &Layer::load_synthetic, py::arg("seed"), py::arg("keep_prob"), py::arg("sigma") = 0.02f,
             py::arg("tail_q") = 0.5f)
        .def("get_scale_rank", &Layer::get_scale_rank)
        .def("set_scale_rank", &Layer::set_scale_rank)
        .def("set_value_scale_raw", &Layer::set_value_scale_raw)
        .def("set_output_scale_raw", &Layer::set_output_scale_raw)
        .def("set_value_scale_raw_k", &Layer::set_value_scale_raw_k)
        .def("set_output_scale_raw_k", &Layer::set_output_scale_raw_k)
        .def("set_importance_scale_raw", &Layer::set_importance_scale_raw)
        .def("set_output_importance_scale_raw", &Layer::set_output_importance_scale_raw)
        .def("set_value_scales", &Layer::set_value_scales)
        .def("set_output_scales", &Layer::set_output_scales)
        .def("get_value_scale", &Layer::get_value_scale)
        .def("get_value_scales", &Layer::get_value_scales)
        .def("get_output_scale", &Layer::get_output_scale)
        .def("get_value_scale_k", &Layer::get_value_scale_k)
        .def("get_output_scale_k", &Layer::get_output_scale_k)
        .def("get_importance_scale", &Layer::get_importance_scale)
        .def("get_output_importance_scale", &Layer::get_output_importance_scale)
        .def("get_scale", &Layer::get_scale)
        .def("get_value_scale_importance", &Layer::get_value_scale_importance, py::arg("row"))
        .def("get_output_scale_importance", &Layer::get_output_scale_importance, py::arg("col"))
        .def("get_scale_state", &Layer::get_scale_state)
        .def("set_stochastic_rounding", &Layer::set_stochastic_rounding, py::arg("on"))
        .def("set_update_variant", &Layer::set_update_variant, py::arg("variant"))
        .def("seed_stochastic_rounding", &Layer::seed_stochastic_rounding, py::arg("seed"))
        .def("forward_dense", &Layer::forward_dense, py::arg("x"))
        .def("backward_dense", &Layer::backward_dense, py::arg("dy"), py::arg("learning_rate"),
             py::arg("lr_per_row_nnz") = false, py::arg("damp_by_importance") = true, py::arg("beta2") = 0.999f,
             py::arg("eps") = 1e-8f)
        .def("sampled_gradw", &Layer::sampled_gradw, py::arg("x"), py::arg("dy"))
        .def("forward_sparse", &Layer::forward_sparse, py::arg("ptrs"), py::arg("indices"), py::arg("values"),
             py::arg("batch"))
        .def("backward_sparse", &Layer::backward_sparse, py::arg("x"), py::arg("dy_ptrs"), py::arg("dy_indices"),
             py::arg("dy_values"), py::arg("batch"), py::arg("learning_rate") = 0.01f,
             py::arg("lr_per_row_nnz") = false, py::arg("damp_by_importance") = true, py::arg("beta2") = 0.999f,
             py::arg("eps") = 1e-8f)
        .def("synapto_step", &Layer::synapto_step, py::arg("prune_frac"), py::arg("cand_rows"),
             py::arg("cand_cols"), py::arg("cand_vals"), py::arg("cand_scores") = py::none(),
             py::arg("default_imp_code") = 1)
        .def("compact", &Layer::compact)
        .def("expand_headroom", &Layer::expand_headroom, py::arg("blank_fraction") = 0.2f)
        .def("expand_headroom_to", &Layer::expand_headroom_to, py::arg("min_nnz_per_row"),
             py::arg("blank_fraction") = 0.2f)
        .def("equalizer_step", &Layer::equalizer_step)
        .def("equalize_to_capacity", &Layer::equalize_to_capacity, py::arg("target_elems_per_row"),
             py::arg("target_bytes_per_row") = 0)
        .def("expand_block4_headroom", &Layer::expand_block4_headroom, py::arg("blank_fraction") = 0.2f)
        .def("compact_block4", &Layer::compact_block4)
        .def("export_block4_layout", &Layer::export_block4_layout)
        .def("zero_accum", &Layer::zero_accum)
        .def("info", &Layer::info)
        .def("export_scattered", &Layer::export_scattered)
        .def("export_layout", &Layer::export_layout)
        .def("_store_digest", &Layer::_store_digest)
        .def("export_block4", &Layer::export_block4)
        .def("decode_scattered", &Layer::decode_scattered)
        .def("build_for_index", &Layer::build_for_index, py::arg("group_size") = 16)
        .def("export_block4_packed", &Layer::export_block4_packed)
        .def_property_readonly("block4", py::cpp_function(&Layer::block4, py::keep_alive<0, 1>()))
        .def("export_for_index", &Layer::export_for_index)
        .def("decode_columns", &Layer::decode_columns, py::arg("use_for_index") = 1)
        .def("synchronize", &Layer::synchronize)
        .def_property_readonly("handle", &Layer::handle)
        .def_property_readonly("n_inputs", &Layer::n_inputs)
        .def_property_readonly("n_outputs", &Layer::n_outputs)
        .def_property_readonly("num_cpus", &Layer::num_cpus)
        .def_property_readonly("nnz", &Layer::nnz)
        .def_property_readonly("out_degree", &Layer::out_degree)
        .def("build_probes", &Layer::build_probes, py::arg("k"), py::arg("per_row") = false)
        .def("synap_row_step", &Layer::synap_row_step, py::arg("current_row"), py::arg("importance_cutoff"),
             py::arg("max_row_weights"), py::arg("max_prune_per_step") = 8, py::arg("importance_eps") = 1e-3f)
        .def("synap_step", &Layer::synap_step, py::arg("importance_cutoff"), py::arg("max_row_weights"),
             py::arg("max_prune_per_step") = 8, py::arg("importance_eps") = 1e-3f)
        .def("get_probes", &Layer::get_probes)
        .def_property_readonly("last_input", &Layer::last_input)
        .def_property_readonly("weights_vals", &Layer::weights_vals)
        .def_property_readonly("importance", &Layer::importance)
        .def_property_readonly("indices", &Layer::indices)
        .def_property_readonly("ptrs", &Layer::ptrs)
        .def_property_readonly("neuron_input_accum", &Layer::neuron_input_accum)
        .def_property_readonly("neuron_grad_accum", &Layer::neuron_grad_accum);
    bind_variant<LayerDeterministic>(m, "SparseLinearLayerDeterministic");
    bind_variant<LayerResync>(m, "SparseLinearLayerResync");
    bind_variant<LayerResyncDeterministic>(m, "SparseLinearLayerResyncDeterministic");
    bind_variant<LayerNoScale>(m, "SparseLinearLayerNoScale");
    bind_variant<LayerNoScaleDeterministic>(m, "SparseLinearLayerNoScaleDeterministic");
    m.def("fp4_quantize_array", &fp4_quantize_array, py::arg("vals"), py::arg("device") = 0);
    m.def("dense_to_csr", &dense_to_csr, py::arg("x"), py::arg("threshold") = 1e-4f, py::arg("device") = 0);
    m.def("dense_to_top_k_csr", &dense_to_top_k_csr, py::arg("x"), py::arg("k"), py::arg("num_threads") = 4,
          py::arg("device") = 0);
    m.def(
        "seed_fp4_stochastic_rng",
        [](uint64_t seed) {
            g_seed = seed;
            ++g_seed_epoch;
        },
        py::arg("seed"));
}
