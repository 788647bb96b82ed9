// layer.hpp -- host-side state of one FP4 delta-CSR layer on one GPU.
#pragma once

#include "common.hpp"

#include <algorithm>
#include <array>
#include <cstring>
#include <map>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

namespace sili {

// Owning device buffer; grows, never shrinks (except reset()).
template <typename T>
struct DevBuf {
    T *p = nullptr;
    size_t n = 0;  // capacity in elements
    DevBuf() = default;
    DevBuf(const DevBuf &) = delete;
    DevBuf &operator=(const DevBuf &) = delete;
    DevBuf(DevBuf &&o) noexcept : p(o.p), n(o.n) { o.p = nullptr; o.n = 0; }
    DevBuf &operator=(DevBuf &&o) noexcept {
        if (this != &o) { reset(); p = o.p; n = o.n; o.p = nullptr; o.n = 0; }
        return *this;
    }
    ~DevBuf() { reset(); }
    void reset() {
        if (p) (void)hipFree(p);
        p = nullptr;
        n = 0;
    }
    // Ensure capacity for `count` elements (+ `pad` bytes of slack so vector
    // loads near the end stay in bounds).  Contents are not preserved.
    // A buffer that has to grow again takes 1/8 more than asked, so a store
    // rebuilt at slowly rising sizes is not reallocated every time.
    void ensure(size_t count, size_t pad = 64) {
        size_t want = count + (pad + sizeof(T) - 1) / sizeof(T);
        if (want <= n && p) return;
        if (p) want += want / 8;
        reset();
        SILI_HIP(hipMalloc(reinterpret_cast<void **>(&p), want * sizeof(T)));
        n = want;
    }
    T *get() const { return p; }
};

// Padded stream copy of a scattered store, read by the stream kernels
// (built on first use, dropped when the store is rebuilt).  The store's
// columns are cut into K blocks of cb columns; block k holds, for every row,
// the row's entries with columns in [k*cb, (k+1)*cb) (K = 1: whole rows).
// In a block, row r occupies bytes [pstart, pstart + L) with pstart a
// multiple of 16: zero bytes first (delta 0: entries at shifted column 0),
// then the varints of the shifted columns col - k*cb + 1 (only the first,
// absolute delta differs from the store's).  Shifted column 0 is a zero
// input slot, so the padding entries (value byte 0) contribute exactly 0.
// val[p] is the value byte of the entry whose varint ends at byte p (0
// elsewhere): value bytes run in parallel with index bytes.  Each block's
// bytes start on a window boundary.
struct DStreamBlock {
    int64_t nbytes = 0, nwin = 0, n_ne = 0, c0 = 0, ncols = 0;
    size_t off = 0, ne_off = 0, win_off = 0;  // into idx/val, ne_row/ne_start, win
};
struct DStream {
    bool valid = false;
    bool failed = false;          // too large for the kernels' 31-bit offsets
    int K = 0;
    int64_t cb = 0;
    std::vector<DStreamBlock> blocks;
    DevBuf<uint8_t> idx, val;     // blocks' bytes (+ padding)
    DevBuf<uint32_t> ne_row;      // per block: non-empty rows, ascending
    DevBuf<uint32_t> ne_start;    // per block: their first byte (+ sentinel: block bytes)
    DevBuf<WinDesc> win;          // per block: nwin + 1 (rs_lo indexes the block's ne lists)
};

// Derived group frame-of-reference (FOR) copy of a store's column indices
// (built on request, dropped when the store is rebuilt).  Per row, groups of
// G columns: a tier byte (0/1/2 = 1/2/4 bytes per offset) and G little-endian
// offsets from the group start (the previous group's last column, 0 for a
// row's first group); a short last group repeats its last offset.  The byte
// stream is the reference prototype's format; the per-group arrays are this
// device's index into it, so every column decodes independently.
struct DFor {
    bool valid = false;
    int G = 16;
    int64_t ngroups = 0, nbytes = 0;
    DevBuf<uint32_t> row_group;   // rows+1: first group of each row
    DevBuf<uint32_t> group_pos;   // ngroups+1: byte offset of each group's tier byte
    DevBuf<uint32_t> group_base;  // ngroups: the group start column
    DevBuf<uint32_t> group_elem;  // ngroups+1: entry index of each group's first column
    DevBuf<uint8_t> bytes;
};

// One orientation of the scattered store.
struct DScatter {
    int64_t rows = 0, cols = 0, nnz = 0, nbytes = 0, nseg = 0;
    int64_t n_empty_rows = 0;  // rows holding no synapse
    bool has_split = false;
    DevBuf<uint32_t> byte_start, elem_start;  // rows+1
    DevBuf<uint8_t> idx, val;
    DevBuf<SegDesc> seg;
    DevBuf<uint32_t> split_rows;  // rows with more than one work item
    int64_t n_split = 0;
    DStream stream1, streamK;     // stream copies: whole rows / the last column blocking used
    DFor fidx;                    // FOR copy of the column indices
    // decoded column of every synapse (u16), for the sparse-input forward's
    // random access (built on first use)
    DevBuf<uint8_t> dcol;
    bool dcol_valid = false;
    // the synapses by input slice for the staged-input gather (built on first
    // use): each synapse's column within its slice of slc_w columns, and per
    // row the first synapse of each of the slc_n slices (rows x (slc_n + 1));
    // slc_w == 0: not built
    DevBuf<uint8_t> slc_col;
    DevBuf<uint32_t> slc_off;
    int64_t slc_w = 0, slc_n = 0;
    // column-block copies for gathers whose operand exceeds one XCD's L2:
    // cblk[k] holds every row's entries with columns in [k*cblk_cb, ...),
    // columns relative to the block (built on first use)
    std::vector<DScatter> cblk;
    int64_t cblk_cb = 0;
    // split rows combined in item order by the float4 gather: arrivals per
    // row (rows+1, zero between launches) and per-item partial sums
    // (part_cap floats; empty: combined by atomics)
    DevBuf<uint32_t> split_cnt;
    DevBuf<float> part;
    int64_t part_cap = 0;
    // the work items split into short rows (whole rows of <= SHORT_ROW_BYTES
    // index bytes, packed several to a wave by the float4 gather) and the
    // others, both in store order (built on first use by gather_plan when at
    // least a quarter of the items are short rows; n_sh == 0: not used).
    // n_short_hint: the short rows the last encode counted (kept, as an
    // estimate, through row patches)
    DevBuf<SegDesc> sh_seg, lg_seg;
    int64_t n_sh = 0, n_lg = 0, n_short_hint = 0;
    bool sh_valid = false;
    GatherPlan plan() const {
        GatherPlan p{seg.p, nseg, idx.p, val.p, rows, cols, has_split, split_rows.p, n_split};
        if (has_split && part_cap > 0) {
            p.elem_start = elem_start.p;
            p.split_cnt = split_cnt.p;
            p.part = part.p;
            p.part_cap = part_cap;
        }
        return p;
    }
};

// One orientation of the block4 store.
struct DBlock4 {
    int64_t brows = 0, bcols = 0, ntiles = 0, nbytes = 0, nseg = 0;
    int64_t rows = 0, cols = 0;  // element extents of this orientation
    bool has_split = false;
    DevBuf<uint32_t> byte_start, tile_start;  // brows+1
    DevBuf<uint8_t> idx;
    DevBuf<uint8_t> tiles;                    // 16 * ntiles
    // canonical store only: the reference's tile_is_sparse per tile (the
    // encoding its Block4Store would hold the tile in; the device computes on
    // the dense 16 bytes and packs on export)
    DevBuf<uint8_t> sparse;
    DevBuf<SegDesc> seg;
    // column-block copies (as DScatter::cblk, in block columns of cblk_cbb)
    std::vector<DBlock4> cblk;
    int64_t cblk_cbb = 0;
    // the tiles by column range (built on first use, kept until the structure
    // changes): each tile's block column, and for range x of rng_k and block
    // row br the first tile of the row in that range, rng_start[x*brows + br]
    // (x = rng_k: the row's end)
    DevBuf<uint32_t> rng_col, rng_start;
    int64_t rng_k = 0;
    B4Ranges ranges() const { return B4Ranges{rng_col.p, rng_start.p, rng_k, brows}; }
    Block4Plan plan() const {
        return Block4Plan{seg.p, nseg, idx.p, tiles.p, rows, cols, has_split};
    }
};

// Pinned host memory (hipHostMalloc), readable and writable by kernels: the
// staging area of the synaptogenesis policy's small reads.  Grows, never
// shrinks.
struct PinBuf {
    uint8_t *h = nullptr;
    size_t n = 0;
    PinBuf() = default;
    PinBuf(const PinBuf &) = delete;
    PinBuf &operator=(const PinBuf &) = delete;
    ~PinBuf() {
        if (in_flight) (void)hipEventSynchronize(ev);
        in_flight = false;
        reset();
        if (ev) (void)hipEventDestroy(ev);
    }
    void reset() {
        wait();
        if (h) (void)hipHostFree(h);
        h = nullptr;
        n = 0;
    }
    // A copy queued from this buffer that nothing else waits for: mark()
    // after queueing it, wait() before the host writes the buffer again.
    void mark(hipStream_t st) {
        if (!ev) SILI_HIP(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
        SILI_HIP(hipEventRecord(ev, st));
        in_flight = true;
    }
    void wait() {
        if (in_flight) {
            in_flight = false;
            SILI_HIP(hipEventSynchronize(ev));
        }
    }
    void ensure(size_t bytes) {
        wait();
        if (h && bytes <= n) return;
        const size_t want = std::max<size_t>(bytes + bytes / 2, 1 << 16);
        reset();
        SILI_HIP(hipHostMalloc(reinterpret_cast<void **>(&h), want, hipHostMallocDefault));
        n = want;
    }

   private:
    hipEvent_t ev = nullptr;
    bool in_flight = false;
};

// The second buffer of each array a row patch rewrites (patch.hip): the
// patch writes the new array here, then the two swap.
struct ScatSpare {
    DevBuf<uint32_t> byte_start, elem_start, perm;
    DevBuf<uint8_t> idx, val;
    DevBuf<SegDesc> seg;
};
struct B4Spare {
    DevBuf<uint32_t> byte_start, tile_start, perm;
    DevBuf<uint8_t> idx, tiles, sparse;
    DevBuf<SegDesc> seg;
};

// One row of a store as staged from the device: its byte and element
// extents, its work items [slo, shi), index bytes, element bytes (value bytes
// or 16-byte tiles) and, when asked, flag bytes and permutation values.
struct StagedRow {
    uint32_t row = 0, b0 = 0, b1 = 0, e0 = 0, e1 = 0, slo = 0, shi = 0;
    std::vector<uint8_t> idx, elems, flags;
    std::vector<uint32_t> perm;
};
// A read of some rows of one store orientation: scattered (s) or block4 (b).
struct StageReq {
    const DScatter *s = nullptr;
    const DBlock4 *b = nullptr;
    const uint8_t *flags = nullptr;   // per-element flag bytes to read too (block4 canonical: tile_is_sparse)
    const uint32_t *perm = nullptr;   // per-element permutation values to read too
    std::vector<uint32_t> rows;       // ascending, distinct
    std::vector<StagedRow> out;
};
// The block row a policy call edits, before and after: its scattered rows
// (col, value byte), ascending, and its tiles (block column -> 16 bytes, slot
// lj*4+li, byte (imp<<4)|w, and the tile's tile_is_sparse).
struct PolicyTile {
    std::array<uint8_t, 16> b{};
    uint8_t sparse = 0;
    bool operator==(const PolicyTile &o) const { return b == o.b && sparse == o.sparse; }
    bool operator!=(const PolicyTile &o) const { return !(*this == o); }
};
struct BlockRowState {
    uint32_t br = 0;
    std::vector<std::pair<uint32_t, uint8_t>> rows[4];
    std::map<uint32_t, PolicyTile> tiles;
};
// A block row as staged from the device for the policy: its canonical rows
// and (when the layer has its block4 store) its row of tiles, with the state
// they decode to.
struct StagedBlock {
    std::vector<StagedRow> w;
    bool has_b4 = false;
    StagedRow b;
    BlockRowState state;
};
// A block row the policy has edited but not yet written to the device: its
// device version as staged, and its state now.
struct PendingBlock {
    StagedBlock orig;
    BlockRowState cur;
};

// Per-kernel event timing of one layer (see ProfScope in common.hpp).
struct Profiler {
    bool enabled = false;
    struct Rec {
        std::string name;
        hipEvent_t a, b;
    };
    std::vector<Rec> recs;
    std::vector<hipEvent_t> pool;
    Profiler() = default;
    Profiler(const Profiler &) = delete;
    Profiler &operator=(const Profiler &) = delete;
    ~Profiler() {
        for (auto &r : recs) { (void)hipEventDestroy(r.a); (void)hipEventDestroy(r.b); }
        for (auto e : pool) (void)hipEventDestroy(e);
    }
    hipEvent_t take() {
        if (!pool.empty()) {
            hipEvent_t e = pool.back();
            pool.pop_back();
            return e;
        }
        hipEvent_t e;
        SILI_HIP(hipEventCreate(&e));
        return e;
    }
};

// Makes L's profiler the target of ProfScopes issued by this thread while in
// scope, and names the entry point ("fwd", "bwd", ...).
struct ProfCtx {
    ProfCtx(struct Layer &L, const char *op);
    ~ProfCtx();
    Profiler *prev;
    ProfOp op;
};

// Scratch that device builders need for one call.
struct Scratch {
    DevBuf<uint8_t> temp;    // rocprim temporary storage
    DevBuf<int> flag;        // validation flag
    // rocprim's temporary storage for a call needing `bytes`: when it must
    // grow it takes half again as much, so sorts that grow step by step
    // (a layer whose synapse count rises) reallocate, and wait on hipFree,
    // only every few steps
    void *temp_for(size_t bytes) {
        const size_t need = bytes + 16;
        temp.ensure(temp.p && temp.n < need + 64 ? need + need / 2 : need);
        return temp.p;
    }
};

// The scale-update variants of the reference's layer classes
// (sili/cpu_backend.cpp:992-1013): RMSprop steps on the scales written in the
// loop (SparseLinearLayer), DeferredScaleWrite (SparseLinearLayerResync),
// NoScalePolicy (SparseLinearLayerNoScale).
enum UpdateVariant : int { UPDATE_PLAIN = 0, UPDATE_RESYNC = 1, UPDATE_NOSCALE = 2 };

struct Layer {
    int device = 0;
    hipStream_t stream = nullptr;
    int64_t n_in = 0, n_out = 0, max_weights = 0;
    int64_t idx_budget = 0, val_budget = 0, tile_budget = 0;
    int rank = 1;
    // Set while a step rebuilds the stores from arrays it produced itself
    // (in range and ordered by construction): the builds then skip their
    // input checks' waits on the stream.
    bool trusted_build = false;
    bool vs_ones = true, os_ones = true;  // rank 1 and all ones
    bool output_scale_trainable = false;
    bool has_nonfinite = false;
    bool nonfinite_scales = false;
    DScatter W, Wt;       // canonical, shadow
    DBlock4 B4, B4t;      // canonical, shadow
    DevBuf<float> vs, os, is, ois;
    DevBuf<float> acc_in, acc_grad;
    // per-call workspace (grown on demand)
    DevBuf<float> ws_xT, ws_gT, ws_out;
    DevBuf<float> ws_s0;  // component 0 of rank > 1 scales: value [n_in], then output [n_out]
    DevBuf<float> ws_xs;  // the staged-input gather's column-scaled input copy
    int64_t xT_cached_batch = 0;  // > 0: ws_xT holds the last forward_dense input, feature-major
    Scratch scratch;
    Profiler prof;
    // backward with the optimizer update: the scales' optimizer state
    // (delta_csr_types.hpp:1127-1215), allocated and zeroed on first use
    DevBuf<float> vs_imp, vs_mom, os_imp;  // [n_in*rank], [n_in*rank], [n_out*rank]
    DevBuf<uint32_t> vs_step, os_step;
    bool train_state_ready = false;
    DevBuf<uint32_t> Wt_perm;     // shadow entry -> canonical entry (kept once the layer trains)
    DevBuf<uint32_t> B4t_perm;    // block4 shadow tile -> canonical tile (kept with every block4 build)
    DevBuf<float> b4term;         // per tile slot: output-scale gradient terms of the update
    bool keep_perm = false;
    DevBuf<float> pow_tab;        // pow_tab[s] = powf(beta2, s), s <= pow_n
    int64_t pow_n = 0;
    float pow_beta2 = 0.0f;
    DevBuf<float> mterm;          // per-synapse output-scale gradient terms
    DevBuf<double> dead_S;
    DevBuf<float> def_w, def_i;   // DeferredScaleWrite: true-units (cw, ci) per synapse
    DevBuf<float> vs_snap;        // value scales as the update's rows read them
    DevBuf<double> train_rowsum;  // backward_sparse update: per-row value-scale gradient sums
    int update_variant = UPDATE_PLAIN;
    // the reference's synaptogenesis policy: the probe list (COO, host; the
    // count may be zeroed while the vectors stay, delta_csr_memory.hpp:1338-1342),
    // the synap_step cursor, and out_degree as the policy keeps it (from the
    // first policy step on; before that, the scattered synapses per column)
    std::vector<int32_t> probe_r, probe_c;
    std::vector<float> probe_v;
    int64_t probe_nnz = 0;
    int64_t synap_cursor = 0;
    DevBuf<int32_t> out_deg;
    bool out_deg_tracked = false;
    // Temporaries of the structure rebuild, kept between calls while
    // keep_temps is set (the synaptogenesis policy rebuilds after every edit:
    // allocating and freeing them each call would cost more than the work).
    // They are used on the layer's stream only, in stream order.
    std::unordered_map<std::string, DevBuf<uint8_t>> temps;
    bool keep_temps = false;
    bool stochastic_rounding = true;
    uint64_t rng_seed = 0x5EEDull, rng_calls = 0;
    int64_t train_calls = 0;
    uint32_t switch_point = 10;  // tiles with <= this many live slots are stored sparse-packed
    // The reference's per-row reservations of its scattered store (index
    // bytes, value elements: used + blank, DeltaCSRLayout) and its
    // equalizer_step cursor; the device store itself stays compact.
    std::vector<uint64_t> lay_b, lay_e;
    int64_t eq_cursor = 0;
    // The reference's per-block-row reservations of its block4 store (index
    // bytes, tile slots, tile bytes: block_layout byte_start / elem_start and
    // tile_byte_start), its budgets (max_indices_bytes, max_tile_bytes), its
    // equalize_step cursor and dropped_growth_events.  b4_ta_dev: the tile
    // bytes as the updates' write-back reads them (re-uploaded when stale);
    // b4_ctr: [evicted slots, row_merge_overflow_events, bytes dropped].
    std::vector<uint64_t> b4_ia, b4_ea, b4_ta;
    uint64_t b4_idx_budget = ~0ull, b4_tile_budget = ~0ull;
    int64_t b4_eq_cursor = 0;
    uint64_t b4_dropped = 0;
    bool b4_ta_stale = true;
    DevBuf<uint32_t> b4_ta_dev;
    DevBuf<unsigned long long> b4_ctr;
    PinBuf pin_b4ta;
    uint32_t seg_len = SEG_BYTES_MAX;  // max index bytes per decode work item (scattered)
    uint32_t seg_len_b4 = 128;  // max block-index bytes per decode work item (block4)
    // the policy's row patches: pinned staging (reads in, patch content out),
    // the device copy of the patch content, and the arrays' second buffers
    PinBuf pin_rows, pin_stage, pin_patch, pin_deg, pin_acc;
    PinBuf pin_read;  // ReadBack's staging
    PinBuf pin_bulk;  // BulkRead's staging
    // The activity accumulators as build_probes last staged them (pin_acc),
    // with its top-k selections over them (k, indices), valid while acc_epoch
    // == policy_epoch: no entry point that may change them has run since.
    uint64_t acc_epoch = ~0ull;
    int64_t sel_in_k = -1, sel_out_k = -1;
    std::vector<size_t> sel_in, sel_out;
    // The policy's block rows: staged and unchanged (clean, valid while no
    // entry point that may change the layer has run: policy_epoch), and
    // edited but not yet written (pending, written by policy_flush before any
    // other entry point touches the layer).
    std::map<uint32_t, StagedBlock> policy_clean;
    std::map<uint32_t, PendingBlock> policy_pending;
    uint64_t policy_epoch = 0, clean_epoch = ~0ull;
    DevBuf<uint8_t> patch_blob;
    ScatSpare sp_W, sp_Wt;
    B4Spare sp_B4, sp_B4t;
};

// A temporary device buffer of a structure rebuild: its own allocation, or,
// while L.keep_temps is set, the layer's kept buffer for this call site.
template <typename T>
struct TmpBuf {
    T *p = nullptr;
    TmpBuf(Layer &L, const char *key) : L_(&L), key_(key) {}
    TmpBuf(const TmpBuf &) = delete;
    TmpBuf &operator=(const TmpBuf &) = delete;
    void ensure(size_t count, size_t pad = 64) {
        if (L_->keep_temps) {
            // a kept buffer that must grow takes half again as much: a layer
            // whose synapse count rises step by step reallocates (and, with
            // hipFree, waits for the device) only every few steps
            DevBuf<uint8_t> &b = L_->temps[key_];
            const size_t need = count * sizeof(T) + pad;
            b.ensure(b.p && b.n < need ? need + need / 2 : need, 0);
            p = reinterpret_cast<T *>(b.p);
        } else {
            own_.ensure(count, pad);
            p = own_.p;
        }
    }
   private:
    Layer *L_;
    const char *key_;
    DevBuf<T> own_;
};
#define SILI_STR2(x) #x
#define SILI_STR(x) SILI_STR2(x)
#define SILI_TMPKEY(name) __FILE__ ":" SILI_STR(__LINE__) ":" #name

// ---- builders (build.hip) ---------------------------------------------------
// Encode a store from row-sorted entries: ptrs[rows+1] (device), cols[N]
// (device, strictly increasing within a row, < ncols), value bytes[N].
// Throws SILI_ERR_INVALID on malformed input.
void prepare_split_combine(Layer &L, DScatter &s);
void build_scattered(Layer &L, DScatter &dst, int64_t rows, int64_t ncols, int64_t N,
                     const uint32_t *d_ptrs, const uint32_t *d_cols, const uint8_t *d_bytes);
// Build the shadow (transposed) store of `src` whose decoded entries are
// (d_rows[e], d_cols[e], src.val[e]).
void build_shadow(Layer &L, const DScatter &src, const uint32_t *d_rows, const uint32_t *d_cols,
                  DScatter &dst);
// Block4 store (and its shadow) from an unsorted device tile list.
// d_flags (optional, parallel to the input tiles): the tiles' tile_is_sparse;
// NULL: every tile encoded by its live count (a load).  sorted_head >= 0:
// tiles [0, sorted_head) and [sorted_head, n_tiles) are each in canonical
// (block row, block column) order, and the canonical build merges them.
void build_block4(Layer &L, int64_t n_tiles, const uint32_t *d_br, const uint32_t *d_bc,
                  const uint8_t *d_tiles, const uint8_t *d_flags = nullptr, int64_t sorted_head = -1);
// Full decode of the canonical scattered store into device arrays.
void decode_scattered(Layer &L, uint32_t *d_rows, uint32_t *d_cols);
// Recompute has_nonfinite (code 8 anywhere, or a non-finite scale).
void refresh_nonfinite(Layer &L);

// The reference's scattered layout (layout.hip): per-row content read from
// the device store, reservations kept on the host.
void row_content(Layer &L, std::vector<uint64_t> &bytes, std::vector<uint64_t> &elems);
void layout_from_absolute(Layer &L, float blank_fraction);
void layout_compact(Layer &L);
// min_nnz_per_row < 0: expand_headroom, else expand_headroom_to
void layout_expand(Layer &L, float blank_fraction, int64_t min_nnz_per_row);
void layout_equalize_to_capacity(Layer &L, int64_t target_elems, int64_t target_bytes);
void layout_equalizer_step(Layer &L);
// after a structural change the reference has no counterpart for: rows
// whose content outgrew their reservation get exactly their content
void layout_fit(Layer &L);
void export_layout(Layer &L, uint64_t *byte_start, uint64_t *byte_end, uint64_t *elem_start, uint64_t *elem_end);

// ---- the reference's block4 reservations (b4res.hip) ------------------------
struct B4Use {  // per block row: block-column index bytes, tiles, stored tile bytes
    std::vector<uint64_t> ui, ue, ut;
};
B4Use b4_row_use(Layer &L);
void b4res_reset(Layer &L, uint64_t idx_budget, uint64_t tile_budget);
void b4res_shift(Layer &L, size_t row, uint64_t ti, uint64_t tt, uint64_t te, uint64_t ui, uint64_t ue,
                 uint64_t ut);
void b4res_insert_tile(Layer &L, size_t row, int64_t idx_delta, uint64_t ui, uint64_t ue, uint64_t ut);
bool b4res_commit(Layer &L, size_t row, uint64_t old_len, uint64_t new_len, uint64_t ut);
void b4res_expand(Layer &L, float blank_fraction, uint64_t slack, const std::vector<uint64_t> &ut);
void b4res_load_dense(Layer &L, const std::vector<uint8_t> &live);
void b4res_put_tiles(Layer &L, int64_t n, const uint32_t *br, const uint32_t *bc, const uint8_t *tiles);
void b4res_equalize_step(Layer &L);
void b4res_fit(Layer &L);
const uint32_t *b4res_device_alloc(Layer &L, hipStream_t st);
unsigned long long *b4res_counters(Layer &L, hipStream_t st);
void b4res_read_counters(Layer &L, uint64_t out[3]);

// FOR index of the canonical scattered store (for_index.hip): build (group
// size 8, 16, 32 or 64), and decode of every column into cols (int32, storage
// order) from the FOR copy or, for comparison, from the ULEB128 stream.
// The sparse-input forward over the active (batch row, input row) pairs
// (push.hip): y[b, :] (+)= sum over batch row b's CSR entries (r, x) of
// x * W[r, :].  push_supported: the layer's output row fits a block's LDS.
constexpr size_t PUSH_LDS_MAX = 150 * 1024;
bool push_supported(const Layer &L);
void ensure_decoded_cols(Layer &L, hipStream_t st);
void launch_push_fwd(Layer &L, const int32_t *xptrs, const int32_t *xidx, const float *xval, int64_t B,
                     const ScaleView &sc, float *y, bool add, hipStream_t st);

void build_for_index(Layer &L, int G);
void decode_columns(Layer &L, int32_t *cols, int use_for, hipStream_t st);

// Block4 tile encoding (tile_enc.hip): re-encode tiles by their live count
// (all, or those with dirty[t] != 0); the tiles a sparse-gradient update
// touched (a nonzero dy in one of their columns, gT feature-major [n_out, B]);
// and the reference's stored tile bytes for export.
void tiles_reencode(Layer &L, const uint8_t *dirty, hipStream_t st);
void tiles_reencode_sparse_update(Layer &L, const float *gT, int64_t B, hipStream_t st);
struct PackedTiles {
    std::vector<uint8_t> flags, bytes;
    std::vector<uint64_t> row_start;  // brows + 1
    int64_t live = 0;
};
PackedTiles export_tiles_packed(Layer &L);

// Module CSR utilities (csr_util.hip): device buffers, synchronous on st.
void dense_to_csr_device(const float *x, int64_t rows, int64_t cols, float threshold, int32_t *ptrs, int32_t *idx,
                         float *vals, int64_t cap, int64_t *nnz, hipStream_t st);
void dense_to_top_k_csr_device(const float *x, int64_t rows, int64_t cols, int64_t k, int32_t *ptrs, int32_t *idx,
                               float *vals, int64_t *nnz, hipStream_t st);

// rocprim wrappers
// The plan of a scattered store for a float4 gather over nb batch columns:
// with its short rows split off (built on first use) where that applies.
GatherPlan gather_plan(Layer &L, DScatter &s, int64_t nb);
void device_exclusive_scan_u64(Layer &L, const uint64_t *in, uint64_t *out, int64_t n);
void device_exclusive_scan_u32(Layer &L, const uint32_t *in, uint32_t *out, int64_t n);
// Small device values read back with one stream synchronization: each
// value is copied asynchronously into pinned memory, then one wait, then the
// values are copied out.  (A copy into pageable host memory waits for the
// stream by itself: one round trip per value.)  At most 8 values of up to 64
// bytes each; one ReadBack in flight per layer.
// The values are fetched at wait() by one kernel that writes them into the
// pinned buffer (where a copy per value cost a runtime copy launch each), so
// nothing queued between add() and wait() may change them.
struct ReadBackSrc {
    const void *src[8];
    uint32_t bytes[8];
    int n;
};
void readback_launch(Layer &L, const ReadBackSrc &a);  // build.hip
struct ReadBack {
    Layer &L;
    void *dst[8];
    ReadBackSrc a{};
    explicit ReadBack(Layer &l) : L(l) { L.pin_read.ensure(8 * 64); }
    void add(void *d, const void *src, size_t bytes) {
        if (a.n == 8 || bytes > 64) throw_error(1, "ReadBack: too many or too large values (internal error)");
        dst[a.n] = d;
        a.src[a.n] = src;
        a.bytes[a.n++] = (uint32_t)bytes;
    }
    void wait() {
        if (a.n) readback_launch(L, a);
        SILI_HIP(hipStreamSynchronize(L.stream));
        for (int i = 0; i < a.n; ++i) std::memcpy(dst[i], L.pin_read.h + 64 * i, a.bytes[i]);
        a.n = 0;
    }
};

// Whole device arrays read to the host through pinned memory (L.pin_bulk):
// every copy queued, then one wait.  Destinations are written at wait().
struct BulkRead {
    Layer &L;
    struct Item {
        void *dst;
        const void *src;
        size_t bytes;
    };
    std::vector<Item> items;
    explicit BulkRead(Layer &l) : L(l) {}
    void add(void *dst, const void *src, size_t bytes) {
        if (bytes) items.push_back(Item{dst, src, bytes});
    }
    void wait() {
        size_t total = 0;
        for (const Item &it : items) total += (it.bytes + 15) & ~size_t(15);
        L.pin_bulk.ensure(total);
        size_t off = 0;
        for (const Item &it : items) {
            SILI_HIP(hipMemcpyAsync(L.pin_bulk.h + off, it.src, it.bytes, hipMemcpyDeviceToHost, L.stream));
            off += (it.bytes + 15) & ~size_t(15);
        }
        SILI_HIP(hipStreamSynchronize(L.stream));
        off = 0;
        for (const Item &it : items) {
            std::memcpy(it.dst, L.pin_bulk.h + off, it.bytes);
            off += (it.bytes + 15) & ~size_t(15);
        }
        items.clear();
    }
};

void device_sort_pairs_u32(Layer &L, const uint32_t *kin, uint32_t *kout, const uint32_t *vin,
                           uint32_t *vout, int64_t n, int bits);
void device_sort_pairs_u64(Layer &L, const uint64_t *kin, uint64_t *kout, const uint32_t *vin,
                           uint32_t *vout, int64_t n, int bits);

// Column-block copies of s (s.cblk, K blocks of cb columns; block4: cbb
// block columns).
void build_colblocks(Layer &L, DScatter &s, int K, int64_t cb);
void build_colblocks_b4(Layer &L, DBlock4 &b, int K, int64_t cbb);
// The staged-input gather (staged.hip): whether it takes this case, and
// out[b, r] for every row r of s (written, not added).
bool staged_supported(const Layer &L, const DScatter &s, const ScaleView &sc, const float *in, int64_t B, int skip);
void launch_gather_staged(Layer &L, DScatter &s, const ScaleView &sc, const float *in, int64_t B, float *out,
                          int64_t out_ld, hipStream_t st);
// b.rng_* for K column ranges of ceil(bcols / K) block columns.
void ensure_col_ranges(Layer &L, DBlock4 &b, int K);
// Block4 contribution (added into out) in column-block passes when the
// gathered operand exceeds 4 MiB (slices of SILI_COLBLOCK_B4_MB, default 8);
// false: not applicable (then use launch_gather_b4).
bool gather_b4_colblocked(Layer &L, DBlock4 &b, const ScaleView &sc, const float *in, int64_t B, float *out,
                          int64_t out_ld, int skip, hipStream_t st);
// out[b*out_ld + row] for b < B over s, in column-block passes when the
// gathered operand (s.cols x B fp32) exceeds one XCD's L2 (pass 0 stores, the
// others add; SILI_COLBLOCK=0 disables).  Returns false, launching nothing,
// when the passes do not apply (then use launch_gather).
bool gather_colblocked(Layer &L, DScatter &s, const ScaleView &sc, const float *in, int64_t B, float *out,
                       int64_t out_ld, int skip, hipStream_t st);

// ---- batch-1 stream kernels (stream.hip) ---------------------------------------
// Whether stream_gather serves this call (batch 1, 2, 4 or 8 with the input
// feature-major and unpadded, no skip rule, rank-1 scales; SILI_B1_STREAM:
// 0 never, 1 stores of >= 1 MiB of index bytes (default), 2 always).
bool stream_wanted(const DScatter &s, const ScaleView &sc, int64_t nb, int64_t in_ld, int skip);
// out[b*out_ld + row] = sum_e dec(code_e) * S(row, col_e) * in[col_e*B + b]
// for every row of s and b < B (zeroes out first; builds s.stream on first
// use).
void stream_gather(Layer &L, DScatter &s, const ScaleView &sc, const float *in, int64_t B, float *out,
                   int64_t out_ld, hipStream_t st);

// ---- backward with the optimizer update (train.hip) -------------------------------
// Largest batch of one update call (the per-row dx accumulator lives in LDS).
constexpr int64_t TRAIN_MAX_BATCH = 1024;
struct TrainParams {
    float lr;
    int lr_per_row_nnz, damp_by_importance;
    float beta2, eps, beta1, min_decay_frac, max_abs_delta, max_ci, zero_escape_eps;
};
// Per-synapse update of the canonical store, dx, and the value scales of its
// rows (needs L's train state and pow table).
void launch_train_rows(Layer &L, const float *xT, const float *gT, int64_t B, float *dx, const TrainParams &p,
                       uint64_t seed, hipStream_t st);
// value_scale steps of the rows without synapses.
void launch_train_dead_rows(Layer &L, const float *xT, const float *gT, int64_t B, const TrainParams &p,
                            hipStream_t st);
// output_scale steps (needs L.Wt_perm and L.mterm).
void launch_train_cols(Layer &L, const TrainParams &p, hipStream_t st);
// Shadow value bytes from the canonical ones (needs L.Wt_perm).
void launch_shadow_val_refresh(Layer &L, hipStream_t st);
// DeferredScaleWrite: the value bytes under the final scales (after the
// scale steps; same seed as launch_train_rows).
void launch_train_store(Layer &L, uint64_t seed, hipStream_t st);
// The block4 tiles' update (after launch_train_rows; adds into dx), the
// block rows' scale step; the tiles' output-scale terms into L.b4term when
// the output scales train.
void launch_train_b4(Layer &L, const float *xT, const float *gT, int64_t B, float *dx, const TrainParams &p,
                     uint64_t seed, hipStream_t st);
// Shadow tile bytes from the canonical ones (through L.B4t_perm).
void launch_b4_shadow_refresh(Layer &L, hipStream_t st);
// the dense update's block-row write-back with eviction (merge_row_workspace),
// after the tiles were re-encoded by live count
void launch_b4_merge(Layer &L, hipStream_t st);
// the canonical block4 tiles' block columns (decoded once per structure)
const uint32_t *b4_tile_cols(Layer &L);
// The sparse-gradient update of block4 tiles and their block rows' value-scale step.
void launch_sparse_train_b4(Layer &L, const float *xT, const float *gT, int64_t B, float *dx,
                            const TrainParams &p, uint64_t seed, hipStream_t st);
// backward_sparse's update of the canonical store, dx and the value scales;
// gT dense feature-major with the sparse dy's entries marked (nonzero bits).
void launch_sparse_train(Layer &L, const float *xT, const float *gT, int64_t B, float *dx, const TrainParams &p,
                         hipStream_t st);

// ---- the reference's synaptogenesis policy (policy.hip) -------------------------
// delta_csr_build_probes over L's activity accumulators.
void build_probes(Layer &L, int64_t k, bool per_row);
// delta_csr_synap_row_step on row cursor % n_in (cursor advanced).
bool synap_row_step(Layer &L, int64_t &cursor, float importance_cutoff, int64_t max_row_weights,
                    int64_t max_prune_per_step, float importance_eps);
// out_degree [n_out] to host memory.
void get_out_degree(Layer &L, int32_t *out);

// ---- seeded synthetic layers (gen.hip) ----------------------------------------
// Rebuilds the scattered store (and its shadow) from the seeded generator and
// writes the per-row value scales into L.vs (rank 1).  Returns the synapse count.
int64_t generate_synthetic(Layer &L, uint64_t seed, double keep_prob, float sigma, float tail_q);

// ---- synaptogenesis (synapto.hip) ---------------------------------------------
void synapto_step(Layer &L, float prune_frac, const int32_t *cand_r, const int32_t *cand_c,
                  const float *cand_v, const float *cand_s, int64_t n_cand, int default_imp,
                  int64_t *stats);
// The same pipeline; explicit_prune: instead of the smallest |w|, the n_prune
// stored synapses whose (row << 32 | col) keys prune_keys holds (host memory;
// with PRUNE_TILE set: the synapse's tile slot, for a synapse stored both in
// its row and in a tile) are removed (tiles left with < 2 live slots
// demoted), then every valid candidate is grown (promotion as in
// synapto_step).
constexpr uint64_t PRUNE_TILE = 1ull << 63;
void synapto_apply(Layer &L, float prune_frac, bool explicit_prune, const uint64_t *prune_keys, int64_t n_prune,
                   const int32_t *cand_r, const int32_t *cand_c, const float *cand_v, const float *cand_s,
                   int64_t n_cand, int default_imp, int64_t *stats);

// ---- row patches for the synaptogenesis policy (patch.hip) ----------------------
// Every request in one round trip: the kernels write pinned memory, one sync.
void stage_rows(Layer &L, const std::vector<StageReq *> &reqs);
// acc_in (n_in) then acc_grad (n_out) in pinned memory, valid until the
// next call that stages or patches.
const float *stage_accumulators(Layer &L);
// The columns (block columns) of a staged row, from its ULEB128 deltas.
std::vector<uint32_t> staged_cols(const StagedRow &r);

// Rewrite the stores for block row br going from `old` to `nu`: the changed
// canonical rows and block row, the shadow rows and block rows they touch,
// their work items and the permutations, with the arrays of every other row
// copied over shifted (no sort, no re-encode of unchanged rows).  w_rows: the
// canonical rows of br as staged for `old`; b4_row: block row br as staged
// (NULL when the layer has no block4 store yet).  Returns false, changing
// nothing, when a patch does not apply (then rebuild instead).
bool patch_block_row(Layer &L, const BlockRowState &old, const BlockRowState &nu,
                     const std::vector<StagedRow> &w_rows, const StagedRow *b4_row);
// The pending edits of many block rows at once: the changed canonical rows
// and block rows patched in, then both shadows rebuilt from the canonical
// stores (the device sort and encode every load uses).
void patch_blocks_rebuild_shadows(Layer &L, const std::vector<const PendingBlock *> &blocks);
// Write every pending policy edit to the device (policy.hip).
void policy_flush(Layer &L);

}  // namespace sili
