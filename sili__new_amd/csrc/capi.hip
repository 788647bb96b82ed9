// capi.hip -- the extern "C" boundary (include/sili_hip.h) and the layer's
// host-side orchestration of the kernels.
#include "../../include/sili_hip.h"
#include "layer.hpp"
#include "wave.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <memory>
#include <mutex>
#include <new>
#include <numeric>
#include <stdexcept>
#include <string>
#include <vector>

struct sili_layer {
    sili::Layer L;
};

// The no-allocation forward's scratch: every GPU the library runs on holds its
// own copy until the process ends.
constexpr size_t NOALLOC_SCRATCH_BYTES = size_t(32) << 20;
static __device__ __align__(256) float scratch[NOALLOC_SCRATCH_BYTES / sizeof(float)];

namespace sili {

namespace {
thread_local std::string g_last_error;
thread_local Profiler *t_prof = nullptr;
thread_local const char *t_op = "";
thread_local const char *t_kernel = nullptr;
}  // namespace

ProfOp::ProfOp(const char *op) : prev(t_op) { t_op = op; }
ProfOp::~ProfOp() { t_op = prev; }

ProfScope::ProfScope(const char *kernel, hipStream_t) : prev(t_kernel) { t_kernel = kernel; }
ProfScope::~ProfScope() { t_kernel = prev; }

bool prof_next(hipEvent_t *start, hipEvent_t *stop) {
    if (!t_prof || !t_prof->enabled || !t_kernel) return false;
    Profiler::Rec r{std::string(t_op) + ":" + t_kernel, t_prof->take(), t_prof->take()};
    *start = r.a;
    *stop = r.b;
    t_prof->recs.push_back(std::move(r));
    return true;
}

ProfCtx::ProfCtx(Layer &L, const char *op) : prev(t_prof), op(op) { t_prof = &L.prof; }
ProfCtx::~ProfCtx() { t_prof = prev; }

void throw_error(int code, const std::string &msg) { throw Error{code, msg}; }

void hip_check(hipError_t e, const char *what) {
    if (e != hipSuccess) {
        const int code = (e == hipErrorOutOfMemory) ? SILI_ERR_NOMEM : SILI_ERR_HIP;
        throw Error{code, std::string("HIP error ") + hipGetErrorString(e) + " in " + what};
    }
}

namespace {

template <typename F>
int guarded(F &&f) {
    try {
        f();
        g_last_error.clear();
        return SILI_OK;
    } catch (const Error &e) {
        g_last_error = e.msg;
        return e.code;
    } catch (const std::bad_alloc &) {
        g_last_error = "out of host memory";
        return SILI_ERR_NOMEM;
    } catch (const std::exception &e) {
        g_last_error = e.what();
        return SILI_ERR_RUNTIME;
    }
}

constexpr unsigned TPB = 256;
inline unsigned nblk(int64_t n) { return (unsigned)((n + TPB - 1) / TPB); }

__global__ void k_fill_f32(float *__restrict__ p, int64_t n, float v) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i < n) p[i] = v;
}

// n4 float4 stores (16-byte aligned p)
__global__ void k_fill_f32x4(float4 *__restrict__ p, int64_t n4, float v) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i < n4) p[i] = make_float4(v, v, v, v);
}

__global__ void k_quantize(const float *__restrict__ w, const float *__restrict__ imp, int64_t n,
                           uint8_t *__restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i >= n) return;
    const uint32_t wc = fp4_encode(w[i]);
    const uint32_t ic = imp ? fp4_encode(imp[i]) : 0u;
    out[i] = (uint8_t)((wc << 4) | ic);
}

// fp4_quantize_array: the raw 4-bit code per element (no importance nibble)
__global__ void k_fp4_codes(const float *__restrict__ x, int64_t n, uint8_t *__restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i < n) out[i] = (uint8_t)fp4_encode(x[i]);
}

__global__ void k_i32_to_u32(const int32_t *__restrict__ s, int64_t n, uint32_t *__restrict__ d) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i < n) d[i] = (uint32_t)s[i];
}

void fill(float *p, int64_t n, float v, hipStream_t st) {
    if (n <= 0) return;
    ProfScope ps("fill", st);
    const int64_t n4 = (reinterpret_cast<uintptr_t>(p) & 15u) == 0 ? n / 4 : 0;
    if (n4 > 0) launch(k_fill_f32x4, dim3(nblk(n4)), dim3(TPB), 0, st, reinterpret_cast<float4 *>(p), n4, v);
    if (n - 4 * n4 > 0) launch(k_fill_f32, dim3(nblk(n - 4 * n4)), dim3(TPB), 0, st, p + 4 * n4, n - 4 * n4, v);
    SILI_HIP(hipGetLastError());
}

// n elements of T, then `tail` (< sizeof(T)) single bytes, by a grid-stride
// loop; src or dst may be page-locked host memory, which the device reads or
// writes over the host link.
template <typename T>
__global__ __launch_bounds__(256) void k_copy_vec(const T *__restrict__ src, T *__restrict__ dst, int64_t n,
                                                  const uint8_t *__restrict__ src_tail,
                                                  uint8_t *__restrict__ dst_tail, int tail) {
    const int64_t stride = (int64_t)gridDim.x * TPB;
    for (int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x; i < n; i += stride) dst[i] = src[i];
    if (blockIdx.x == 0 && (int)threadIdx.x < tail) dst_tail[threadIdx.x] = src_tail[threadIdx.x];
}

// Whether `p` is page-locked host memory that the device addresses at the
// same address (hipHostMalloc memory on ROCm).  Pageable memory is not known
// to the runtime: the query fails and its error is cleared.
bool host_locked(const void *p) {
    hipPointerAttribute_t a{};
    if (hipPointerGetAttributes(&a, p) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    return a.type == hipMemoryTypeHost && a.devicePointer == p;
}

// A copy between device memory and page-locked host memory as one kernel on
// `st`.  The runtime's DMA copies on a stream have been measured at about a
// quarter of their usual rate (2 MiB in 0.15-0.2 ms against 0.045 ms) on
// streams of a process after a large layer was built, and staying so; the
// kernel moves 2 MiB in about 0.05 ms on any stream.  Up to 128 blocks of
// 32 KiB each per pass (the host link, not the grid, bounds it).
void kernel_copy(void *dst, const void *src, size_t bytes, hipStream_t st) {
    const uintptr_t al = reinterpret_cast<uintptr_t>(dst) | reinterpret_cast<uintptr_t>(src);
    auto go = [&](auto tag) {
        using T = decltype(tag);
        const int64_t n = (int64_t)(bytes / sizeof(T));
        const int tail = (int)(bytes - (size_t)n * sizeof(T));
        const unsigned grid = (unsigned)std::min<int64_t>(128, std::max<int64_t>(1, (n + 2047) / 2048));
        ProfScope ps("copy_host", st);
        launch(k_copy_vec<T>, dim3(grid), dim3(TPB), 0, st, static_cast<const T *>(src), static_cast<T *>(dst), n,
               static_cast<const uint8_t *>(src) + (size_t)n * sizeof(T),
               static_cast<uint8_t *>(dst) + (size_t)n * sizeof(T), tail);
    };
    if ((al & 15u) == 0) go(uint4{});
    else if ((al & 3u) == 0) go(uint32_t{});
    else go(uint8_t{});
    SILI_HIP(hipGetLastError());
}

// Every entry point that reaches a layer's device state comes here first.
// The policy's own (policy = true) leave its pending edits pending; any
// other writes them first and, unless it only reads the layer
// (set_device_read), ends the validity of what the policy has staged (its
// block rows, the accumulators and their top-k selections).
void set_device(Layer &L, bool policy = false) {
    SILI_HIP(hipSetDevice(L.device));
    if (!policy) {
        if (!L.policy_pending.empty()) policy_flush(L);
        ++L.policy_epoch;
    }
}
// Entry points that change nothing of the layer's stores or accumulators.
void set_device_read(Layer &L) {
    SILI_HIP(hipSetDevice(L.device));
    if (!L.policy_pending.empty()) policy_flush(L);
}
// Readers of the scales only (no store access).
void set_device(const Layer &L) { SILI_HIP(hipSetDevice(L.device)); }

// Scratch of sili_forward_dense_noalloc (the file-scope array `scratch`):
// host code never names the array in a kernel argument or a copy, it uses the
// per-device address that hipGetSymbolAddress returns, resolved once per
// device at the first sili_create on that device, with the device current.
constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
float *g_scratch_ptr[MAX_DEVICES] = {};

void resolve_scratch(int device) {
    if (device < 0 || device >= MAX_DEVICES) throw_error(SILI_ERR_INVALID, "device ordinal out of range");
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (g_scratch_ptr[device]) return;
    void *ptr = nullptr;
    SILI_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
    g_scratch_ptr[device] = static_cast<float *>(ptr);
}

float *scratch_on(int device) {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    return (device >= 0 && device < MAX_DEVICES) ? g_scratch_ptr[device] : nullptr;
}

hipStream_t pick(const Layer &L, void *stream) {
    return stream ? reinterpret_cast<hipStream_t>(stream) : L.stream;
}

template <typename T>
void upload(DevBuf<T> &dst, const T *src, size_t n, hipStream_t st) {
    dst.ensure(n);
    if (n) SILI_HIP(hipMemcpyAsync(dst.p, src, n * sizeof(T), hipMemcpyHostToDevice, st));
}

// Canonical scales: rows index vs, entries index os.  Shadow: the reverse.
ScaleView canon_scales(const Layer &L) {
    if (L.rank == 1) return ScaleView{L.vs_ones ? nullptr : L.vs.p, L.os_ones ? nullptr : L.os.p, 1};
    return ScaleView{L.vs.p, L.os.p, L.rank};
}
ScaleView shadow_scales(const Layer &L) {
    if (L.rank == 1) return ScaleView{L.os_ones ? nullptr : L.os.p, L.vs_ones ? nullptr : L.vs.p, 1};
    return ScaleView{L.os.p, L.vs.p, L.rank};
}

// The sparse-input forward and the sparse-gradient backward read component 0
// of every scale only, whatever the rank: stored * (vs[r,0] * os[c,0])
// (sisldo_ops.hpp:302-306,527-531 and the lr == 0 dx of
// disldo_backward_sparse_grad).  A rank > 1 layer's component 0 is strided,
// so it is gathered into a rank-1 pair first.
__global__ void k_scale_comp0(const float *__restrict__ vs, const float *__restrict__ os, int64_t n_in,
                              int64_t n_out, int rank, float *__restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * TPB + threadIdx.x;
    if (i < n_in) out[i] = vs[i * rank];
    else if (i < n_in + n_out) out[i] = os[(i - n_in) * rank];
}
ScaleView comp0_scales(Layer &L, bool shadow, hipStream_t st) {
    if (L.rank == 1) return shadow ? shadow_scales(L) : canon_scales(L);
    L.ws_s0.ensure((size_t)(L.n_in + L.n_out));
    launch(k_scale_comp0, dim3(nblk(L.n_in + L.n_out)), dim3(TPB), 0, st, (const float *)L.vs.p,
           (const float *)L.os.p, L.n_in, L.n_out, L.rank, L.ws_s0.p);
    SILI_HIP(hipGetLastError());
    const float *v0 = L.ws_s0.p, *o0 = L.ws_s0.p + L.n_in;
    return shadow ? ScaleView{o0, v0, 1} : ScaleView{v0, o0, 1};
}

void rebuild_shadow(Layer &L) {
    DevBuf<uint32_t> rows, cols;
    rows.ensure((size_t)L.W.nnz + 1);
    cols.ensure((size_t)L.W.nnz + 1);
    decode_scattered(L, rows.p, cols.p);
    build_shadow(L, L.W, rows.p, cols.p, L.Wt);
}

void build_from_host_csr(Layer &L, const int32_t *ptrs, const int32_t *idx, const uint8_t *bytes_h,
                         const float *w_h, const float *imp_h, int64_t nnz) {
    if (!ptrs) throw_error(SILI_ERR_INVALID, "load_weights: ptrs is NULL");
    if (nnz < 0 || nnz >= (int64_t(1) << 31)) throw_error(SILI_ERR_INVALID, "load_weights: nnz out of range");
    if (ptrs[0] != 0 || ptrs[L.n_in] != nnz)
        throw_error(SILI_ERR_INVALID, "load_weights: ptrs[0] must be 0 and ptrs[n_inputs] must equal nnz");
    for (int64_t r = 0; r < L.n_in; ++r)
        if (ptrs[r + 1] < ptrs[r]) throw_error(SILI_ERR_INVALID, "load_weights: ptrs must be non-decreasing");
    if (nnz > 0 && (!idx || (!bytes_h && !w_h)))
        throw_error(SILI_ERR_INVALID, "load_weights: indices/values missing");
    // reference budgets grow to fit a load (sili/cpu_backend.cpp:866-872)
    L.idx_budget = std::max<int64_t>(L.idx_budget, nnz * 8 + 4096);
    L.val_budget = std::max<int64_t>(L.val_budget, nnz + 64);
    hipStream_t st = L.stream;
    DevBuf<int32_t> dptrs_i, didx_i;
    DevBuf<uint32_t> dptrs, dcols;
    DevBuf<uint8_t> dbytes;
    DevBuf<float> dw, dimp;
    upload(dptrs_i, ptrs, (size_t)L.n_in + 1, st);
    dptrs.ensure((size_t)L.n_in + 1);
    launch(k_i32_to_u32, dim3(nblk(L.n_in + 1)), dim3(TPB), 0, st, dptrs_i.p, L.n_in + 1, dptrs.p);
    dcols.ensure((size_t)nnz + 1);
    dbytes.ensure((size_t)nnz + 1);
    if (nnz > 0) {
        upload(didx_i, idx, (size_t)nnz, st);
        launch(k_i32_to_u32, dim3(nblk(nnz)), dim3(TPB), 0, st, didx_i.p, nnz, dcols.p);
        if (bytes_h) {
            SILI_HIP(hipMemcpyAsync(dbytes.p, bytes_h, (size_t)nnz, hipMemcpyHostToDevice, st));
        } else {
            upload(dw, w_h, (size_t)nnz, st);
            if (imp_h) upload(dimp, imp_h, (size_t)nnz, st);
            launch(k_quantize, dim3(nblk(nnz)), dim3(TPB), 0, st, dw.p, imp_h ? dimp.p : nullptr,
                               nnz, dbytes.p);
        }
        SILI_HIP(hipGetLastError());
    }
    // negative indices become huge u32 values and fail the range check
    build_scattered(L, L.W, L.n_in, L.n_out, nnz, dptrs.p, dcols.p, dbytes.p);
    rebuild_shadow(L);
    refresh_nonfinite(L);
    // delta_csr_from_absolute's reservations, blank_fraction 0.2
    // (sili/cpu_backend.cpp:873-874, and the constructor's empty layer)
    layout_from_absolute(L, 0.2f);
}

void empty_stores(Layer &L) {
    std::vector<int32_t> p((size_t)L.n_in + 1, 0);
    build_from_host_csr(L, p.data(), nullptr, nullptr, nullptr, nullptr, 0);
    build_block4(L, 0, nullptr, nullptr, nullptr);
}

void check_scales_finite(Layer &L, const std::vector<float> &vs, const std::vector<float> &os) {
    bool bad = false;
    for (float v : vs) bad |= !std::isfinite(v);
    for (float v : os) bad |= !std::isfinite(v);
    L.nonfinite_scales = bad;
}

void refresh_scale_flags(Layer &L) {
    std::vector<float> vs((size_t)L.n_in * L.rank), os((size_t)L.n_out * L.rank);
    SILI_HIP(hipMemcpyAsync(vs.data(), L.vs.p, vs.size() * 4, hipMemcpyDeviceToHost, L.stream));
    SILI_HIP(hipMemcpyAsync(os.data(), L.os.p, os.size() * 4, hipMemcpyDeviceToHost, L.stream));
    SILI_HIP(hipStreamSynchronize(L.stream));
    L.vs_ones = L.rank == 1 && std::all_of(vs.begin(), vs.end(), [](float v) { return v == 1.0f; });
    L.os_ones = L.rank == 1 && std::all_of(os.begin(), os.end(), [](float v) { return v == 1.0f; });
    check_scales_finite(L, vs, os);
    refresh_nonfinite(L);
}

void reset_scales(Layer &L) {
    // component 0 defaults to 1, k >= 1 to 0 (delta_csr_types.hpp:1116-1121)
    std::vector<float> vs((size_t)L.n_in * L.rank, 0.0f), os((size_t)L.n_out * L.rank, 0.0f);
    for (int64_t r = 0; r < L.n_in; ++r) vs[(size_t)r * L.rank] = 1.0f;
    for (int64_t c = 0; c < L.n_out; ++c) os[(size_t)c * L.rank] = 1.0f;
    upload(L.vs, vs.data(), vs.size(), L.stream);
    upload(L.os, os.data(), os.size(), L.stream);
    SILI_HIP(hipStreamSynchronize(L.stream));
    L.vs_ones = L.os_ones = (L.rank == 1);
    L.nonfinite_scales = false;
    L.train_state_ready = false;  // the scales' optimizer state restarts at zero
}

// Feature-major copy of activations [B, n] -> [n, B] (B == 1: no copy).
const float *to_feature_major(Layer &L, DevBuf<float> &ws, const float *x, int64_t B, int64_t n,
                              float *acc, hipStream_t st) {
    if (B == 1) {
        if (acc) launch_colabs(x, 1, n, acc, st);
        return x;
    }
    ws.ensure((size_t)(n * B));
    launch_transpose(x, B, n, ws.p, acc, st);
    return ws.p;
}

inline bool al16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// The independent small tasks an entry point issues before its gathers,
// collected and run in one launch (k_prep); a task whose shape the fused
// kernel does not take is launched on its own at once (it is independent
// of the others).
struct Prep {
    PrepTask t[PREP_MAX];
    int n = 0;
    hipStream_t st;
    explicit Prep(hipStream_t s) : st(s) {}
    bool room() const { return n < PREP_MAX; }
    void add(int kind, const float *src, float *dst, float *acc, int64_t B, int64_t cnt, int64_t ld = 0,
             const uint32_t *rows = nullptr, float v = 0.0f) {
        t[n++] = PrepTask{kind, 0u, src, dst, acc, B, cnt, ld, rows, v};
    }
    // feature-major copy [B, n] -> [n, B] (B == 1: none), sum |.| into acc
    const float *feature_major(DevBuf<float> &ws, const float *x, int64_t B, int64_t cols, float *acc) {
        if (B == 1) {
            if (acc) colabs(x, 1, cols, acc);
            return x;
        }
        ws.ensure((size_t)(cols * B));
        if (room() && B % 4 == 0 && cols % 4 == 0 && al16(x) && al16(ws.p)) add(PREP_TRANSPOSE, x, ws.p, acc, B, cols);
        else launch_transpose(x, B, cols, ws.p, acc, st);
        return ws.p;
    }
    void colabs(const float *x, int64_t B, int64_t cols, float *acc) {
        if (room() && cols % 4 == 0 && al16(x) && al16(acc)) add(PREP_COLABS, x, nullptr, acc, B, cols);
        else launch_colabs(x, B, cols, acc, st);
    }
    void rowabs(const float *xT, int64_t B, int64_t cols, float *acc) {
        if (room()) add(PREP_ROWABS, xT, nullptr, acc, B, cols);
        else launch_rowabs(xT, B, cols, acc, st);
    }
    void fill(float *p, int64_t cnt, float v) {
        const int64_t n4 = al16(p) ? cnt / 4 : 0;
        if (n4 > 0 && room()) {
            add(PREP_FILL4, nullptr, p, nullptr, 0, n4, 0, nullptr, v);
            if (cnt - 4 * n4 > 0) ::sili::fill(p + 4 * n4, cnt - 4 * n4, v, st);
        } else {
            ::sili::fill(p, cnt, v, st);
        }
    }
    // out[b, row] = 0 for every split row (launch_zero_split_rows' rule)
    void zero_split(const GatherPlan &p, float *out, int64_t ld, int64_t nb) {
        if (p.nseg == 0 || nb == 0 || !p.has_split || p.n_split == 0) return;
        if (p.n_split * 4 >= p.rows) fill(out, nb * ld, 0.0f);
        else if (room()) add(PREP_ZERO_LIST, nullptr, out, nullptr, nb, p.n_split, ld, p.split_rows);
        else launch_zero_split_rows(p, out, ld, nb, st);
    }
    void run() {
        launch_prep(t, n, st);
        n = 0;
    }
};

}  // namespace

// Column-block passes of a scattered gather over s, or 0 when they do not
// apply.  SILI_COLBLOCK (read per call): 0 never, else when the gathered
// operand is larger than 4 MiB (one XCD's L2); passes of <= SILI_COLBLOCK_MB
// (default 2 MiB: measured on c4's down layer at batch 128, 8 passes of
// 2 MiB beat 4 of 4 MiB and 2 of 8 MiB).
int64_t colblock_passes(const DScatter &s, const float *in, int64_t B) {
    const int mode = env_int("SILI_COLBLOCK", 1);
    if (mode == 0 || s.nnz == 0 || B % 4 != 0 || B > 512 || (reinterpret_cast<uintptr_t>(in) & 15u) != 0) return 0;
    const int64_t opbytes = s.cols * B * 4;
    if (opbytes <= (int64_t(4) << 20) || opbytes >= (int64_t)0x80000000LL) return 0;
    const int64_t slice = (int64_t)std::max(1, env_int("SILI_COLBLOCK_MB", 2)) << 20;
    const int64_t K = std::min<int64_t>(16, (opbytes + slice - 1) / slice);
    return K < 2 ? 0 : K;
}

bool gather_colblocked(Layer &L, DScatter &s, const ScaleView &sc, const float *in, int64_t B, float *out,
                       int64_t out_ld, int skip, hipStream_t st) {
    const int64_t K = colblock_passes(s, in, B);
    if (K == 0) return false;
    const int64_t cb = (s.cols + K - 1) / K;
    if ((int64_t)s.cblk.size() != K || s.cblk_cb != cb) build_colblocks(L, s, (int)K, cb);
    for (int64_t k = 0; k < K; ++k) {
        DScatter &sub = s.cblk[(size_t)k];
        const int64_t c0 = k * cb;
        const ScaleView sk{sc.row, sc.ent ? sc.ent + c0 * sc.rank : nullptr, sc.rank};
        // pass 0 stores (split rows zeroed first), later passes add
        if (k == 0) launch_zero_split_rows(sub.plan(), out, out_ld, B, st);
        launch_gather(sub.plan(), sk, in + c0 * B, B, out, out_ld, B, skip, st, k > 0);
    }
    return true;
}

bool gather_b4_colblocked(Layer &L, DBlock4 &b, const ScaleView &sc, const float *in, int64_t B, float *out,
                          int64_t out_ld, int skip, hipStream_t st) {
    // as gather_colblocked; the block4 gathers add into out, so every pass
    // adds.  Slices of SILI_COLBLOCK_B4_MB (default 8 MiB: measured on c3,
    // 2 passes of 8 MiB beat 4 of 4 MiB, 8 of 2 MiB and one of 16 MiB; shorter
    // block rows per pass cost more than the cache misses they save)
    const int mode = env_int("SILI_COLBLOCK", 1);
    if (mode == 0 || b.ntiles == 0 || skip != SKIP_NONE || B % 4 != 0 ||
        (reinterpret_cast<uintptr_t>(in) & 15u) != 0)
        return false;
    const int64_t opbytes = b.cols * B * 4;
    if (opbytes <= (int64_t(4) << 20) || opbytes >= (int64_t)0x80000000LL) return false;
    const int64_t slice = (int64_t)std::max(1, env_int("SILI_COLBLOCK_B4_MB", 8)) << 20;
    const int64_t K = std::min<int64_t>(16, (opbytes + slice - 1) / slice);
    if (K < 2) return false;
    const int64_t cbb = (b.bcols + K - 1) / K;
    if ((int64_t)b.cblk.size() != K || b.cblk_cbb != cbb) build_colblocks_b4(L, b, (int)K, cbb);
    for (int64_t k = 0; k < K; ++k) {
        const int64_t c0 = k * cbb * 4;
        const ScaleView sk{sc.row, sc.ent ? sc.ent + c0 * sc.rank : nullptr, sc.rank};
        launch_gather_b4(b.cblk[(size_t)k].plan(), sk, in + c0 * B, B, out, out_ld, B, skip, st);
    }
    return true;
}

namespace {

void forward_dense(Layer &L, const float *x, int64_t B, float *y, hipStream_t st) {
    ProfCtx pc(L, "fwd");
    if (B <= 0) throw_error(SILI_ERR_INVALID, "forward_dense: batch must be >= 1");
    if (!x || !y) throw_error(SILI_ERR_INVALID, "forward_dense: NULL buffer");
    // the input's feature-major copy and the output's zeroing in one launch
    Prep prep(st);
    const float *xT = prep.feature_major(L.ws_xT, x, B, L.n_in, nullptr);
    // the feature-major copy doubles as the stored forward input that
    // backward_dense reads when called without x (sili/cpu_backend.cpp:481)
    L.xT_cached_batch = B > 1 ? B : 0;
    // scattered pass skips exact-zero inputs (linear_disldo.hpp:114); only
    // observable with non-finite weights, so the skip is compiled in only then
    const int skip = L.has_nonfinite ? SKIP_ZERO : SKIP_NONE;
    const ScaleView ssc = shadow_scales(L);
    const bool str = L.Wt.nnz > 0 && stream_wanted(L.Wt, ssc, B, B, skip);
    // batches 65..128: the input staged in LDS slice by slice (SILI_STAGED)
    const bool staged = L.Wt.nnz > 0 && !str && env_int("SILI_STAGED", 1) && staged_supported(L, L.Wt, ssc, xT, B, skip);
    const bool plain = L.Wt.nnz > 0 && !str && !staged && colblock_passes(L.Wt, xT, B) == 0;
    if (L.Wt.nnz == 0) prep.fill(y, B * L.n_out, 0.0f);
    else if (plain) prep.zero_split(L.Wt.plan(), y, L.n_out, B);
    prep.run();
    if (str) stream_gather(L, L.Wt, ssc, xT, B, y, L.n_out, st);
    else if (staged) launch_gather_staged(L, L.Wt, ssc, xT, B, y, L.n_out, st);
    else if (plain) launch_gather(gather_plan(L, L.Wt, B), ssc, xT, B, y, L.n_out, B, skip, st);
    else if (L.Wt.nnz > 0 && !gather_colblocked(L, L.Wt, ssc, xT, B, y, L.n_out, skip, st))
        throw_error(SILI_ERR_RUNTIME, "forward_dense: column-block passes did not apply (internal error)");
    if (L.B4t.ntiles > 0 && !gather_b4_colblocked(L, L.B4t, shadow_scales(L), xT, B, y, L.n_out, SKIP_NONE, st))
        launch_gather_b4(L.B4t.plan(), shadow_scales(L), xT, B, y, L.n_out, B, SKIP_NONE, st);
}

// forward_dense without device allocation: the feature-major copy of x goes
// to the per-device scratch, and only structures built at load are read (the
// segment gathers over the shadow stores: no stream or column-block copies,

// The block4 sampled grad-W by column range: ceil(gT bytes / 4 MiB) ranges
// (at most 8), so that each XCD's L2 (4 MiB) holds its range's gT rows
// (SILI_SDDMM_RANGES: the number of ranges, 0 for the store's work items).
void sddmm_b4(Layer &L, const float *xT, const float *gT, int64_t B, float *gw, hipStream_t st) {
    const int64_t gT_bytes = L.B4.cols * B * 4, l2 = int64_t(4) << 20;
    const int K = env_int("SILI_SDDMM_RANGES", (int)std::min<int64_t>(8, std::max<int64_t>(1, (gT_bytes + l2 - 1) / l2)));
    if (K >= 1) {
        ensure_col_ranges(L, L.B4, K);
        const B4Ranges r = L.B4.ranges();
        launch_sddmm_b4(L.B4.plan(), &r, xT, gT, B, gw, st);
    } else {
        launch_sddmm_b4(L.B4.plan(), nullptr, xT, gT, B, gw, st);
    }
}

// which are built on first use).  No profiler context, so no events either.
void forward_dense_noalloc(Layer &L, const float *x, int64_t B, float *y, hipStream_t st) {
    if (B <= 0) throw_error(SILI_ERR_INVALID, "forward_dense_noalloc: batch must be >= 1");
    if (!x || !y) throw_error(SILI_ERR_INVALID, "forward_dense_noalloc: NULL buffer");
    if (B > 1 && (uint64_t)L.n_in * (uint64_t)B > NOALLOC_SCRATCH_BYTES / sizeof(float))
        throw_error(SILI_ERR_INVALID, "forward_dense_noalloc: n_inputs * batch exceeds the scratch of " +
                                          std::to_string(NOALLOC_SCRATCH_BYTES / sizeof(float)) + " floats");
    float *scr = scratch_on(L.device);
    if (!scr) throw_error(SILI_ERR_RUNTIME, "forward_dense_noalloc: scratch not resolved on this device");
    const float *xT = x;
    if (B > 1) {
        launch_transpose(x, B, L.n_in, scr, nullptr, st);
        xT = scr;
    }
    // the stored forward input (ws_xT) no longer belongs to the last forward
    L.xT_cached_batch = 0;
    const int skip = L.has_nonfinite ? SKIP_ZERO : SKIP_NONE;
    const ScaleView ssc = shadow_scales(L);
    if (L.Wt.nnz == 0) {
        fill(y, B * L.n_out, 0.0f, st);
    } else {
        launch_zero_split_rows(L.Wt.plan(), y, L.n_out, B, st);
        launch_gather(L.Wt.plan(), ssc, xT, B, y, L.n_out, B, skip, st);
    }
    if (L.B4t.ntiles > 0) launch_gather_b4(L.B4t.plan(), ssc, xT, B, y, L.n_out, B, SKIP_NONE, st);
}

void backward_dense(Layer &L, const float *x, const float *dy, int64_t B, float *dx, float *gw_s,
                    float *gw_b, hipStream_t st) {
    ProfCtx pc(L, "bwd");
    if (B <= 0) throw_error(SILI_ERR_INVALID, "backward_dense: batch must be >= 1");
    if (!dy || !dx) throw_error(SILI_ERR_INVALID, "backward_dense: NULL buffer");
    const bool want_gw = gw_s || gw_b;
    // the feature-major copies, the accumulators' sums and dx's zeroing in
    // one launch
    Prep prep(st);
    const float *xT = nullptr;
    if (!x) {
        if (L.xT_cached_batch != B)
            throw_error(SILI_ERR_INVALID, "backward_dense: x is NULL but no forward_dense input of this batch "
                                          "(> 1) is stored; pass x");
        xT = L.ws_xT.p;
    } else if (want_gw) {
        xT = prep.feature_major(L.ws_xT, x, B, L.n_in, nullptr);
        L.xT_cached_batch = 0;
    }
    // accumulators always advance (linear_disldo.hpp:515-520); sum|x| rides
    // on the grad-W kernel when it runs
    const float *gT = prep.feature_major(L.ws_gT, dy, B, L.n_out, L.acc_grad.p);
    const bool scat = L.W.nnz > 0;
    // sum|x| rides on the scattered grad-W kernel when that runs (a copy of x
    // made in this launch is summed from x itself)
    if (!(scat && gw_s)) {
        if (xT && xT == L.ws_xT.p && x == nullptr) prep.rowabs(xT, B, L.n_in, L.acc_in.p);
        else prep.colabs(x, B, L.n_in, L.acc_in.p);
    }
    // grad-input and grad-W read the same gT row per synapse: one fused pass
    // when grad-W is wanted; otherwise the stream kernels (small batches) or
    // the segment gather
    const bool str = scat && !gw_s && stream_wanted(L.W, canon_scales(L), B, B, SKIP_NONE);
    if (!scat) prep.fill(dx, B * L.n_in, 0.0f);
    else if (!str) prep.zero_split(L.W.plan(), dx, L.n_in, B);
    prep.run();
    const bool fused = scat && gw_s &&
                       launch_bwd_fused(L.W.plan(), canon_scales(L), gT, xT, B, dx, L.n_in, gw_s, L.acc_in.p, st);
    if (str) stream_gather(L, L.W, canon_scales(L), gT, B, dx, L.n_in, st);
    else if (scat && !fused && !gather_colblocked(L, L.W, canon_scales(L), gT, B, dx, L.n_in, SKIP_NONE, st))
        launch_gather(gather_plan(L, L.W, B), canon_scales(L), gT, B, dx, L.n_in, B, SKIP_NONE, st);
    if (L.B4.ntiles > 0 && !gather_b4_colblocked(L, L.B4, canon_scales(L), gT, B, dx, L.n_in, SKIP_NONE, st))
        launch_gather_b4(L.B4.plan(), canon_scales(L), gT, B, dx, L.n_in, B, SKIP_NONE, st);
    if (scat && gw_s && !fused) launch_sddmm(L.W.plan(), xT, gT, B, gw_s, L.acc_in.p, st);
    if (gw_b && L.B4.ntiles > 0) sddmm_b4(L, xT, gT, B, gw_b, st);
}

// The scales' optimizer state, zeroed on first use (the reference sizes it
// with zeros inside disldo_backward, linear_disldo.hpp:578-605).
void ensure_train_state(Layer &L, hipStream_t st) {
    if (L.train_state_ready) return;
    const size_t nr = (size_t)(L.n_in * L.rank), nc = (size_t)(L.n_out * L.rank);
    L.vs_imp.ensure(nr);
    L.vs_mom.ensure(nr);
    L.vs_step.ensure(nr);
    L.os_imp.ensure(nc);
    L.os_step.ensure(nc);
    fill(L.vs_imp.p, (int64_t)nr, 0.0f, st);
    fill(L.vs_mom.p, (int64_t)nr, 0.0f, st);
    fill(reinterpret_cast<float *>(L.vs_step.p), (int64_t)nr, 0.0f, st);
    fill(L.os_imp.p, (int64_t)nc, 0.0f, st);
    fill(reinterpret_cast<float *>(L.os_step.p), (int64_t)nc, 0.0f, st);
    L.train_state_ready = true;
}

// pow_tab[s] = powf(beta2, s) for s <= need: the bias correction of
// RMSpropScalePolicy::update (delta_csr_types.hpp:427), computed with the
// host's powf (the function the reference calls) and looked up on the device.
void ensure_pow_table(Layer &L, float beta2, int64_t need, hipStream_t st) {
    if (L.pow_n >= need && std::memcmp(&L.pow_beta2, &beta2, 4) == 0 && L.pow_tab.p) return;
    const int64_t n = std::max<int64_t>(need, std::max<int64_t>(1024, 2 * L.pow_n));
    std::vector<float> t((size_t)n + 1);
    for (int64_t s = 0; s <= n; ++s) t[(size_t)s] = std::pow(beta2, static_cast<float>(s));
    L.pow_tab.ensure(t.size());
    SILI_HIP(hipMemcpyAsync(L.pow_tab.p, t.data(), t.size() * 4, hipMemcpyHostToDevice, st));
    SILI_HIP(hipStreamSynchronize(st));
    L.pow_n = n;
    L.pow_beta2 = beta2;
}

// The shadow's permutation (shadow entry -> canonical entry): kept from the
// first update on, by rebuilding the shadow once.
void ensure_shadow_perm(Layer &L) {
    if (L.keep_perm && (L.Wt_perm.p || L.W.nnz == 0)) return;
    L.keep_perm = true;
    rebuild_shadow(L);
}

uint64_t splitmix64_host(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// backward_dense with the optimizer update (sili/cpu_backend.cpp:496-529,
// linear_disldo.hpp:466-2113) on a layer without block4 tiles.
void backward_dense_train(Layer &L, const float *x, const float *dy, int64_t B, float *dx, const TrainParams &p,
                          hipStream_t st) {
    ProfCtx pc(L, "bwd");
    if (B <= 0) throw_error(SILI_ERR_INVALID, "backward_dense: batch must be >= 1");
    if (!dy || !dx) throw_error(SILI_ERR_INVALID, "backward_dense: NULL buffer");
    if (B > TRAIN_MAX_BATCH)
        throw_error(SILI_ERR_INVALID, "backward_dense with learning_rate != 0: batch must be <= 1024");
    const float *xT = nullptr;
    if (!x) {
        if (L.xT_cached_batch != B)
            throw_error(SILI_ERR_INVALID, "backward_dense: x is NULL but no forward_dense input of this batch "
                                          "(> 1) is stored; pass x");
        xT = L.ws_xT.p;
    } else {
        xT = to_feature_major(L, L.ws_xT, x, B, L.n_in, nullptr, st);
        L.xT_cached_batch = 0;
    }
    // accumulators (linear_disldo.hpp:515-520)
    const float *gT = to_feature_major(L, L.ws_gT, dy, B, L.n_out, L.acc_grad.p, st);
    launch_rowabs(xT, B, L.n_in, L.acc_in.p, st);
    ensure_train_state(L, st);
    // a value scale's counter steps at most twice per call (the scattered
    // row's step, then its block row's)
    ensure_pow_table(L, p.beta2, 2 * (L.train_calls + 1) + 1, st);
    ensure_shadow_perm(L);
    if (L.output_scale_trainable) L.mterm.ensure((size_t)(L.W.nnz * 2 * L.rank));
    const uint64_t seed = splitmix64_host(L.rng_seed ^ splitmix64_host(L.rng_calls + 1));
    launch_train_rows(L, xT, gT, B, dx, p, seed, st);
    // block4 tiles after the scattered rows' scale steps (linear_disldo.hpp:962-1951)
    launch_train_b4(L, xT, gT, B, dx, p, seed, st);
    // the update rewrites every tile: each is re-encoded by its live count
    // (linear_disldo.hpp:1839-1856, block4.hpp:1336-1355), then each block
    // row is written back, evicting where it outgrew its reservation
    tiles_reencode(L, nullptr, st);
    launch_b4_merge(L, st);
    if (L.W.n_empty_rows > 0) launch_train_dead_rows(L, xT, gT, B, p, st);
    const bool scales_step = L.update_variant != UPDATE_NOSCALE;
    if (L.output_scale_trainable && scales_step && L.W.nnz > 0) launch_train_cols(L, p, st);
    launch_train_store(L, seed, st);
    launch_shadow_val_refresh(L, st);
    launch_b4_shadow_refresh(L, st);
    // copies holding value bytes are stale now: rebuilt on their next use
    for (DScatter *sc : {&L.W, &L.Wt}) {
        sc->stream1.valid = sc->streamK.valid = false;
        sc->cblk.clear();
        sc->cblk_cb = 0;
    }
    for (DBlock4 *b4 : {&L.B4, &L.B4t}) {
        b4->cblk.clear();
        b4->cblk_cbb = 0;
    }
    L.vs_ones = false;
    if (L.output_scale_trainable && scales_step) L.os_ones = false;
    ++L.train_calls;
    ++L.rng_calls;
}

void forward_sparse(Layer &L, const int32_t *ptrs, const int32_t *idx, const float *vals, int64_t nnz_x,
                    int64_t B, float *y, hipStream_t st) {
    ProfCtx pc(L, "fwd_sparse");
    if (B <= 0) throw_error(SILI_ERR_INVALID, "forward_sparse: batch must be >= 1");
    if (!ptrs || !y) throw_error(SILI_ERR_INVALID, "forward_sparse: NULL buffer");
    L.xT_cached_batch = 0;
    // only the active rows of each batch row contribute (sisldo_ops.hpp:271-313).
    // Sparse inputs are pushed from the canonical store (work ~ the active
    // synapse visits); denser ones take the shadow gather (work ~ nnz * B),
    // which is faster above ~2 % active inputs on MI355X (config-2 layer:
    // push 21.3 / 25.7 / 37.8 / 76.8 us at 0.5 / 1 / 3 / 10 %, densify +
    // gather ~32.5 us at any density).
    // SILI_PUSH: 0 never, 2 whenever supported, else below 2 % active pairs.
    const int push_mode = env_int("SILI_PUSH", 1);
    const bool sparse_enough = (double)nnz_x < 0.02 * (double)B * (double)L.n_in;
    const bool push = push_supported(L) && push_mode != 0 && (push_mode == 2 || sparse_enough);
    if (push) launch_push_fwd(L, ptrs, idx, vals, B, comp0_scales(L, false, st), y, false, st);
    if (!push || L.B4t.ntiles > 0) {
        L.ws_xT.ensure((size_t)(L.n_in * B));
        launch_densify_full(ptrs, idx, vals, B, L.n_in, L.ws_xT.p, nullptr, true, nnz_x, st);
    }
    const ScaleView ssc = comp0_scales(L, true, st);
    if (!push) {
        launch_zero_split_rows(L.Wt.plan(), y, L.n_out, B, st);
        launch_gather(gather_plan(L, L.Wt, B), ssc, L.ws_xT.p, B, y, L.n_out, B, SKIP_POSZERO, st);
    }
    if (L.B4t.ntiles > 0) launch_gather_b4(L.B4t.plan(), ssc, L.ws_xT.p, B, y, L.n_out, B, SKIP_POSZERO, st);
}

void backward_sparse(Layer &L, const float *x, const int32_t *dptrs, const int32_t *didx,
                     const float *dvals, int64_t nnz_dy, int64_t B, float *dx, hipStream_t st) {
    ProfCtx pc(L, "bwd_sparse");
    if (B <= 0) throw_error(SILI_ERR_INVALID, "backward_sparse: batch must be >= 1");
    if (!x || !dptrs || !dx) throw_error(SILI_ERR_INVALID, "backward_sparse: NULL buffer");
    launch_colabs(x, B, L.n_in, L.acc_in.p, st);
    L.ws_gT.ensure((size_t)(L.n_out * B));
    launch_densify_full(dptrs, didx, dvals, B, L.n_out, L.ws_gT.p, L.acc_grad.p, true, nnz_dy, st);
    launch_zero_split_rows(L.W.plan(), dx, L.n_in, B, st);
    // scattered: merge-join visits only present dy entries (sisldo_ops.hpp:705-713);
    // block4: skips dy == 0 per slot (sisldo_ops.hpp:886-897)
    const ScaleView csc = comp0_scales(L, false, st);
    launch_gather(gather_plan(L, L.W, B), csc, L.ws_gT.p, B, dx, L.n_in, B, SKIP_POSZERO, st);
    if (L.B4.ntiles > 0) launch_gather_b4(L.B4.plan(), csc, L.ws_gT.p, B, dx, L.n_in, B, SKIP_ZERO, st);
}

// backward_sparse with the optimizer update (sili/cpu_backend.cpp:587-603,
// sisldo_ops.hpp:589-848) on a layer without block4 tiles.
void backward_sparse_train(Layer &L, const float *x, const int32_t *dptrs, const int32_t *didx,
                           const float *dvals, int64_t nnz_dy, int64_t B, float *dx, const TrainParams &p,
                           hipStream_t st) {
    ProfCtx pc(L, "bwd_sparse");
    if (B <= 0) throw_error(SILI_ERR_INVALID, "backward_sparse: batch must be >= 1");
    if (!x || !dptrs || !dx) throw_error(SILI_ERR_INVALID, "backward_sparse: NULL buffer");
    if (B > TRAIN_MAX_BATCH)
        throw_error(SILI_ERR_INVALID, "backward_sparse with learning_rate != 0: batch must be <= 1024");
    const float *xT = to_feature_major(L, L.ws_xT, x, B, L.n_in, nullptr, st);
    L.xT_cached_batch = 0;
    launch_rowabs(xT, B, L.n_in, L.acc_in.p, st);
    L.ws_gT.ensure((size_t)(L.n_out * B));
    // entries present in dy carry nonzero bits (explicit zeros as -0.0)
    launch_densify_full(dptrs, didx, dvals, B, L.n_out, L.ws_gT.p, L.acc_grad.p, true, nnz_dy, st);
    ensure_train_state(L, st);
    // a value scale's counter steps at most twice per call (the scattered
    // row's step, then its block row's)
    ensure_pow_table(L, p.beta2, 2 * (L.train_calls + 1) + 1, st);
    ensure_shadow_perm(L);
    launch_sparse_train(L, xT, L.ws_gT.p, B, dx, p, st);
    // block4 tiles after the scattered section (sisldo_ops.hpp:848-1100)
    const uint64_t seed = splitmix64_host(L.rng_seed ^ splitmix64_host(L.rng_calls + 1));
    // (it re-encodes the tiles it rewrites by their live count and writes
    // each block row back, with eviction, after every batch row,
    // sisldo_ops.hpp:945-1052)
    launch_sparse_train_b4(L, xT, L.ws_gT.p, B, dx, p, seed, st);
    launch_shadow_val_refresh(L, st);
    launch_b4_shadow_refresh(L, st);
    for (DScatter *sc : {&L.W, &L.Wt}) {
        sc->stream1.valid = sc->streamK.valid = false;
        sc->cblk.clear();
        sc->cblk_cb = 0;
    }
    for (DBlock4 *b4 : {&L.B4, &L.B4t}) {
        b4->cblk.clear();
        b4->cblk_cbb = 0;
    }
    L.vs_ones = false;
    ++L.train_calls;
    ++L.rng_calls;
}

void export_block4_coords(Layer &L, std::vector<uint32_t> &br, std::vector<uint32_t> &bc) {
    const int64_t n = L.B4.ntiles;
    br.assign((size_t)n, 0);
    bc.assign((size_t)n, 0);
    if (n == 0) return;
    DevBuf<uint32_t> dbr, dbc;
    dbr.ensure((size_t)n);
    dbc.ensure((size_t)n);
    launch_decode_b4(L.B4.plan(), dbr.p, dbc.p, L.stream);
    SILI_HIP(hipMemcpyAsync(br.data(), dbr.p, (size_t)n * 4, hipMemcpyDeviceToHost, L.stream));
    SILI_HIP(hipMemcpyAsync(bc.data(), dbc.p, (size_t)n * 4, hipMemcpyDeviceToHost, L.stream));
    SILI_HIP(hipStreamSynchronize(L.stream));
}

}  // namespace
}  // namespace sili

using namespace sili;

extern "C" {

const char *sili_last_error(void) { return g_last_error.c_str(); }

int sili_create(int64_t n_inputs, int64_t n_outputs, int64_t max_weights, int device, sili_layer **out) {
    return guarded([&] {
        if (!out) throw_error(SILI_ERR_INVALID, "out is NULL");
        *out = nullptr;
        if (n_inputs <= 0 || n_outputs <= 0 || n_inputs >= (int64_t(1) << 31) || n_outputs >= (int64_t(1) << 31))
            throw_error(SILI_ERR_INVALID, "n_inputs and n_outputs must be in [1, 2^31)");
        if (max_weights < 0) throw_error(SILI_ERR_INVALID, "max_weights must be >= 0");
        auto h = std::make_unique<sili_layer>();
        Layer &L = h->L;
        L.device = device;
        set_device(L);
        resolve_scratch(device);
        SILI_HIP(hipStreamCreateWithFlags(&L.stream, hipStreamNonBlocking));
        L.n_in = n_inputs;
        L.n_out = n_outputs;
        L.max_weights = max_weights;
        // budgets of sili/cpu_backend.cpp:371-373,391-393
        L.idx_budget = max_weights * 8 + 4096;
        L.val_budget = max_weights + 64;
        L.tile_budget = std::max<int64_t>(4, max_weights / 16) * 16;
        // the block4 store's budgets (sili/cpu_backend.cpp:438-441), nothing reserved
        b4res_reset(L, (uint64_t)max_weights * 8 + 4096, (uint64_t)L.tile_budget);
        // segment byte limits (tuning knobs; the kernels stage at most SEG_BYTES_MAX)
        if (const char *e = std::getenv("SILI_SEG_BYTES"))
            L.seg_len = (uint32_t)std::min<int>((int)SEG_BYTES_MAX, std::max(16, std::atoi(e)));
        if (const char *e = std::getenv("SILI_SEG_BYTES_B4"))
            L.seg_len_b4 = (uint32_t)std::min<int>((int)SEG_BYTES_MAX, std::max(16, std::atoi(e)));
        reset_scales(L);
        std::vector<float> ones_in((size_t)n_inputs, 1.0f), ones_out((size_t)n_outputs, 1.0f);
        upload(L.is, ones_in.data(), ones_in.size(), L.stream);
        upload(L.ois, ones_out.data(), ones_out.size(), L.stream);
        L.acc_in.ensure((size_t)n_inputs);
        L.acc_grad.ensure((size_t)n_outputs);
        fill(L.acc_in.p, n_inputs, 0.0f, L.stream);
        fill(L.acc_grad.p, n_outputs, 0.0f, L.stream);
        empty_stores(L);
        SILI_HIP(hipStreamSynchronize(L.stream));
        *out = h.release();
    });
}

void sili_destroy(sili_layer *layer) {
    if (!layer) return;
    (void)hipSetDevice(layer->L.device);
    (void)hipStreamSynchronize(layer->L.stream);
    hipStream_t s = layer->L.stream;
    delete layer;
    if (s) (void)hipStreamDestroy(s);
}

int sili_synchronize(sili_layer *layer) {
    return guarded([&] {
        if (!layer) throw_error(SILI_ERR_INVALID, "layer is NULL");
        set_device_read(layer->L);
        SILI_HIP(hipStreamSynchronize(layer->L.stream));
    });
}

void *sili_stream(sili_layer *layer) { return layer ? reinterpret_cast<void *>(layer->L.stream) : nullptr; }

int sili_load_weights(sili_layer *layer, const int32_t *ptrs, const int32_t *indices, const float *vals,
                      const float *imp, int64_t nnz) {
    return guarded([&] {
        if (!layer) throw_error(SILI_ERR_INVALID, "layer is NULL");
        layer->L.out_deg_tracked = false;  // a load counts out_degree afresh
        set_device(layer->L);
        build_from_host_csr(layer->L, ptrs, indices, nullptr, vals, imp, nnz);
    });
}

int sili_load_weight_bytes(sili_layer *layer, const int32_t *ptrs, const int32_t *indices,
                           const uint8_t *bytes, int64_t nnz) {
    return guarded([&] {
        if (!layer) throw_error(SILI_ERR_INVALID, "layer is NULL");
        layer->L.out_deg_tracked = false;  // a load counts out_degree afresh
        set_device(layer->L);
        if (nnz > 0 && !bytes) throw_error(SILI_ERR_INVALID, "bytes is NULL");
        std::vector<uint8_t> dummy(1, 0);
        build_from_host_csr(layer->L, ptrs, indices, nnz > 0 ? bytes : dummy.data(), nullptr, nullptr, nnz);
    });
}

int sili_load_synthetic(sili_layer *layer, uint64_t seed, double keep_prob, float sigma, float tail_q,
                        int64_t *nnz_out) {
    return guarded([&] {
        if (!layer) throw_error(SILI_ERR_INVALID, "layer is NULL");
        layer->L.out_deg_tracked = false;  // a load counts out_degree afresh
        Layer &L = layer->L;
        if (L.rank != 1) throw_error(SILI_ERR_INVALID, "load_synthetic: scale rank must be 1");
        if (!(keep_prob >= 0.0 && keep_prob <= 1.0) || !(sigma > 0.0f) || !(tail_q >= 0.5f && tail_q < 1.0f))
            throw_error(SILI_ERR_INVALID, "load_synthetic: need 0 <= keep_prob <= 1, sigma > 0, 0.5 <= tail_q < 1");
        set_device(L);
        const int64_t nnz = generate_synthetic(L, seed, keep_prob, sigma, tail_q);
        refresh_scale_flags(L);
        layout_from_absolute(L, 0.2f);  // reserved as load_weights reserves
        if (nnz_out) *nnz_out = nnz;
    });
}

int sili_load_dense_codes(sili_layer *layer, const uint8_t *wc, const uint8_t *ic) {
    return guarded([&] {
        if (!layer) throw_error(SILI_ERR_INVALID, "layer is NULL");
        layer->L.out_deg_tracked = false;  // a load counts out_degree afresh
        if (!wc || !ic) throw_error(SILI_ERR_INVALID, "code arrays are NULL");
        Layer &L = layer->L;
        set_device(L);
        const int64_t brows = (L.n_in + 3) / 4, bcols = (L.n_out + 3) / 4;
        const int64_t n = brows * bcols;
        std::vector<uint32_t> br((size_t)n), bc((size_t)n);
        std::vector<uint8_t> tiles((size_t)n * 16, 0);
        // delta_csr_memory.hpp:884-911: every 4x4 block becomes a tile,
        // slot byte = w | (imp << 4)
        for (int64_t i = 0; i < brows; ++i)
            for (int64_t j = 0; j < bcols; ++j) {
                const int64_t t = i * bcols + j;
                br[(size_t)t] = (uint32_t)i;
                bc[(size_t)t] = (uint32_t)j;
                for (int li = 0; li < 4; ++li)
                    for (int lj = 0; lj < 4; ++lj) {
                        const int64_t r = i * 4 + li, c = j * 4 + lj;
                        if (r >= L.n_in || c >= L.n_out) continue;
                        const size_t k = (size_t)(r * L.n_out + c);
                        tiles[(size_t)t * 16 + (size_t)(lj * 4 + li)] = (uint8_t)(wc[k] | (ic[k] << 4));
                    }
            }
        // the reservations block4_load_dense leaves (delta_csr_memory.hpp:
        // 841-945): new budgets, every tile committed, 20 % headroom
        std::vector<uint8_t> live((size_t)n, 0);
        for (int64_t t = 0; t < n; ++t)
            for (int sl = 0; sl < 16; ++sl) live[(size_t)t] += tiles[(size_t)t * 16 + (size_t)sl] != 0;
        b4res_load_dense(L, live);
        DevBuf<uint32_t> dbr, dbc;
        DevBuf<uint8_t> dt;
        upload(dbr, br.data(), br.size(), L.stream);
        upload(dbc, bc.data(), bc.size(), L.stream);
        upload(dt, tiles.data(), tiles.size(), L.stream);
        build_block4(L, n, dbr.p, dbc.p, dt.p);
        refresh_nonfinite(L);
    });
}

int sili_load_block4_tiles(sili_layer *layer, const int32_t *br, const int32_t *bc, const uint8_t *tile_bytes,
                           int64_t n_tiles) {
    return guarded([&] {
        if (!layer) throw_error(SILI_ERR_INVALID, "layer is NULL");
        layer->L.out_deg_tracked = false;  // a load counts out_degree afresh
        Layer &L = layer->L;
        set_device(L);
        if (n_tiles < 0 || n_tiles >= (int64_t(1) << 31)) throw_error(SILI_ERR_INVALID, "n_tiles out of range");
        if (n_tiles > 0 && (!br || !bc || !tile_bytes)) throw_error(SILI_ERR_INVALID, "tile arrays are NULL");
        std::vector<uint32_t> ubr((size_t)n_tiles), ubc((size_t)n_tiles);
        const int64_t brows = (L.n_in + 3) / 4, bcols = (L.n_out + 3) / 4;
        for (int64_t i = 0; i < n_tiles; ++i) {
            if (br[i] < 0 || bc[i] < 0) throw_error(SILI_ERR_INVALID, "negative tile coordinate");
            if (br[i] >= brows || bc[i] >= bcols)
                throw_error(SILI_ERR_INVALID, "block4 tiles: malformed input (unsorted, duplicate or out-of-range index)");
            ubr[(size_t)i] = (uint32_t)br[i];
            ubc[(size_t)i] = (uint32_t)bc[i];
        }
        // the store's reservations as the tiles placed one by one in
        // canonical order through get_or_create and a handle's writes leave
        // them (block4.hpp:1170-1183,1226-1290): refused with MemoryError,
        // before any device work, where the budget would refuse a row's
        // growth or drop a tile's content
        {
            std::vector<uint32_t> ord((size_t)n_tiles);
            std::iota(ord.begin(), ord.end(), 0u);
            std::sort(ord.begin(), ord.end(), [&](uint32_t a, uint32_t b) {
                return ubr[a] != ubr[b] ? ubr[a] < ubr[b] : ubc[a] < ubc[b];
            });
            std::vector<uint32_t> sbr((size_t)n_tiles), sbc((size_t)n_tiles);
            std::vector<uint8_t> st((size_t)n_tiles * 16);
            for (int64_t i = 0; i < n_tiles; ++i) {
                const uint32_t k = ord[(size_t)i];
                sbr[(size_t)i] = ubr[k];
                sbc[(size_t)i] = ubc[k];
                if (i > 0 && sbr[(size_t)i] == sbr[(size_t)i - 1] && sbc[(size_t)i] == sbc[(size_t)i - 1])
                    throw_error(SILI_ERR_INVALID, "block4 tiles: duplicate entries");
                std::memcpy(&st[(size_t)i * 16], tile_bytes + (size_t)k * 16, 16);
            }
            const auto ia = L.b4_ia, ea = L.b4_ea, ta = L.b4_ta;
            const uint64_t dropped = L.b4_dropped;
            try {
                b4res_reset(L, L.b4_idx_budget, L.b4_tile_budget);
                b4res_put_tiles(L, n_tiles, sbr.data(), sbc.data(), st.data());
            } catch (...) {
                L.b4_ia = ia;
                L.b4_ea = ea;
                L.b4_ta = ta;
                L.b4_dropped = dropped;
                L.b4_ta_stale = true;
                throw;
            }
        }
        DevBuf<uint32_t> dbr, dbc;
        DevBuf<uint8_t> dt;
        upload(dbr, ubr.data(), ubr.size(), L.stream);
        upload(dbc, ubc.data(), ubc.size(), L.stream);
        upload(dt, tile_bytes, (size_t)n_tiles * 16, L.stream);
        build_block4(L, n_tiles, dbr.p, dbc.p, dt.p);
        refresh_nonfinite(L);
    });
}

int sili_set_scale_rank(sili_layer *layer, int rank) {
    return guarded([&] {
        if (!layer) throw_error(SILI_ERR_INVALID, "layer is NULL");
        // sili/cpu_backend.cpp:455-461
        if (rank < 1) throw_error(SILI_ERR_INVALID, "scale_rank must be >= 1");
        if (rank > 4) throw_error(SILI_ERR_INVALID, "scale_rank exceeds SCALE_RANK_MAX (4)");
        Layer &L = layer->L;
        set_device(L);
        L.rank = rank;
        reset_scales(L);
        refresh_nonfinite(L);
    });
}

int sili_get_scale_rank(const sili_layer *layer) { return layer ? layer->L.rank : 0; }

static int set_scale_impl(sili_layer *layer, const float *v, int which) {
    return guarded([&] {
        if (!layer || !v) throw_error(SILI_ERR_INVALID, "NULL argument");
        Layer &L = layer->L;
        set_device(L);
        switch (which) {
            case 0: upload(L.vs, v, (size_t)(L.n_in * L.rank), L.stream); break;
            case 1:
                upload(L.os, v, (size_t)(L.n_out * L.rank), L.stream);
                L.output_scale_trainable = true;
                break;
            case 2: upload(L.is, v, (size_t)L.n_in, L.stream); break;
            default: upload(L.ois, v, (size_t)L.n_out, L.stream); break;
        }
        if (which <= 1) refresh_scale_flags(L);
        else SILI_HIP(hipStreamSynchronize(L.stream));
    });
}

int sili_set_value_scale(sili_layer *layer, const float *vs) { return set_scale_impl(layer, vs, 0); }
int sili_set_output_scale(sili_layer *layer, const float *os) { return set_scale_impl(layer, os, 1); }
int sili_set_importance_scale(sili_layer *layer, const float *is) { return set_scale_impl(layer, is, 2); }
int sili_set_output_importance_scale(sili_layer *layer, const float *ois) { return set_scale_impl(layer, ois, 3); }

static int get_scale_impl(const sili_layer *layer, float *out, bool value) {
    return guarded([&] {
        if (!layer || !out) throw_error(SILI_ERR_INVALID, "NULL argument");
        const Layer &L = layer->L;
        set_device(L);
        const size_t n = (size_t)((value ? L.n_in : L.n_out) * L.rank);
        SILI_HIP(hipMemcpyAsync(out, value ? L.vs.p : L.os.p, n * 4, hipMemcpyDeviceToHost, L.stream));
        SILI_HIP(hipStreamSynchronize(L.stream));
    });
}
int sili_get_value_scale(const sili_layer *layer, float *vs) { return get_scale_impl(layer, vs, true); }
int sili_get_output_scale(const sili_layer *layer, float *os) { return get_scale_impl(layer, os, false); }

int sili_forward_dense(sili_layer *layer, const float *x, int64_t batch, float *y, void *stream) {
    return guarded([&] {
        if (!layer) throw_error(SILI_ERR_INVALID, "layer is NULL");
        set_device(layer->L);
        forward_dense(layer->L, x, batch, y, pick(layer->L, stream));
    });
}

int sili_forward_dense_noalloc(sili_layer *layer, const float *x, int64_t batch, float *y, void *stream) {
    return guarded([&] {
        if (!layer) throw_error(SILI_ERR_INVALID, "layer is NULL");
        // writing the policy's pending edits allocates: refused here rather
        // than done (any other entry point, sili_synchronize included, writes
        // them); the call only reads the layer, so the policy's caches stay
        SILI_HIP(hipSetDevice(layer->L.device));
        if (!layer->L.policy_pending.empty())
            throw_error(SILI_ERR_INVALID, "forward_dense_noalloc: the layer holds pending synaptogenesis policy "
                                          "edits, and writing them allocates; call sili_synchronize first");
        forward_dense_noalloc(layer->L, x, batch, y, pick(layer->L, stream));
    });
}

int sili_backward_dense(sili_layer *layer, const float *x, const float *dy, int64_t batch, float *dx,
                        float *gw_s, float *gw_b, float learning_rate, void *stream) {
    return guarded([&] {
        if (!layer) throw_error(SILI_ERR_INVALID, "layer is NULL");
        set_device(layer->L);
        if (learning_rate != 0.0f) {
            if (gw_s || gw_b)
                throw_error(SILI_ERR_INVALID, "backward_dense: the sampled grad-W is for learning_rate == 0");
            // the reference binding's defaults (sili/cpu_backend.cpp:496-528)
            const TrainParams p{learning_rate, 0, 1, 0.999f, 1e-8f, 0.9f, 0.0f, 2.0f, 100.0f, 0.1f};
            backward_dense_train(layer->L, x, dy, batch, dx, p, pick(layer->L, stream));
            return;
        }
        backward_dense(layer->L, x, dy, batch, dx, gw_s, gw_b, pick(layer->L, stream));
    });
}

int sili_backward_dense_train(sili_layer *layer, const float *x, const float *dy, int64_t batch, float *dx,
                              float learning_rate, int lr_per_row_nnz, int damp_by_importance, float beta2,
                              float eps, void *stream) {
    return guarded([&] {
        if (!layer) throw_error(SILI_ERR_INVALID, "layer is NULL");
        set_device(layer->L);
        hipStream_t st = pick(layer->L, stream);
        if (learning_rate == 0.0f) {
            backward_dense(layer->L, x, dy, batch, dx, nullptr, nullptr, st);
            return;
        }
        const TrainParams p{learning_rate, lr_per_row_nnz ? 1 : 0, damp_by_importance ? 1 : 0, beta2, eps,
                            0.9f, 0.0f, 2.0f, 100.0f, 0.1f};
        backward_dense_train(layer->L, x, dy, batch, dx, p, st);
    });
}

int sili_set_update_variant(sili_layer *layer, int variant) {
    return guarded([&] {
        if (!layer) throw_error(SILI_ERR_INVALID, "layer is NULL");
        if (variant < UPDATE_PLAIN || variant > UPDATE_NOSCALE)
            throw_error(SILI_ERR_INVALID, "update variant must be 0 (plain), 1 (resync) or 2 (noscale)");
        layer->L.update_variant = variant;
    });
}

int sili_set_stochastic_rounding(sili_layer *layer, int on) {
    return guarded([&] {
        if (!layer) throw_error(SILI_ERR_INVALID, "layer is NULL");
        layer->L.stochastic_rounding = on != 0;
    });
}

int sili_seed_stochastic_rounding(sili_layer *layer, uint64_t seed) {
    return guarded([&] {
        if (!layer) throw_error(SILI_ERR_INVALID, "layer is NULL");
        layer->L.rng_seed = seed;
        layer->L.rng_calls = 0;
    });
}

int sili_get_scale_state(const sili_layer *layer, float *vs_importance, float *os_importance, float *vs_momentum,
                         uint32_t *vs_step, uint32_t *os_step) {
    return guarded([&] {
        if (!layer) throw_error(SILI_ERR_INVALID, "layer is NULL");
        const Layer &L = layer->L;
        set_device(L);
        const size_t nr = (size_t)(L.n_in * L.rank), nc = (size_t)(L.n_out * L.rank);
        if (!L.train_state_ready) {
            if (vs_importance) std::fill(vs_importance, vs_importance + nr, 0.0f);
            if (vs_momentum) std::fill(vs_momentum, vs_momentum + nr, 0.0f);
            if (vs_step) std::fill(vs_step, vs_step + nr, 0u);
            if (os_importance) std::fill(os_importance, os_importance + nc, 0.0f);
            if (os_step) std::fill(os_step, os_step + nc, 0u);
            return;
        }
        if (vs_importance) SILI_HIP(hipMemcpyAsync(vs_importance, L.vs_imp.p, nr * 4, hipMemcpyDeviceToHost, L.stream));
        if (vs_momentum) SILI_HIP(hipMemcpyAsync(vs_momentum, L.vs_mom.p, nr * 4, hipMemcpyDeviceToHost, L.stream));
        if (vs_step) SILI_HIP(hipMemcpyAsync(vs_step, L.vs_step.p, nr * 4, hipMemcpyDeviceToHost, L.stream));
        if (os_importance) SILI_HIP(hipMemcpyAsync(os_importance, L.os_imp.p, nc * 4, hipMemcpyDeviceToHost, L.stream));
        if (os_step) SILI_HIP(hipMemcpyAsync(os_step, L.os_step.p, nc * 4, hipMemcpyDeviceToHost, L.stream));
        SILI_HIP(hipStreamSynchronize(L.stream));
    });
}

int sili_sampled_gradw(sili_layer *layer, const float *x, const float *dy, int64_t batch, float *gw_s,
                       float *gw_b, void *stream) {
    return guarded([&] {
        if (!layer) throw_error(SILI_ERR_INVALID, "layer is NULL");
        Layer &L = layer->L;
        if (batch <= 0 || !x || !dy) throw_error(SILI_ERR_INVALID, "sampled_gradw: bad arguments");
        set_device(L);
        ProfCtx pc(L, "gradw");
        hipStream_t st = pick(L, stream);
        const float *xT = to_feature_major(L, L.ws_xT, x, batch, L.n_in, nullptr, st);
        L.xT_cached_batch = 0;
        const float *gT = to_feature_major(L, L.ws_gT, dy, batch, L.n_out, nullptr, st);
        if (gw_s) launch_sddmm(L.W.plan(), xT, gT, batch, gw_s, nullptr, st);
        if (gw_b && L.B4.ntiles > 0) sddmm_b4(L, xT, gT, batch, gw_b, st);
    });
}

int sili_forward_sparse(sili_layer *layer, const int32_t *ptrs, const int32_t *indices, const float *values,
                        int64_t nnz_x, int64_t batch, float *y, void *stream) {
    return guarded([&] {
        if (!layer) throw_error(SILI_ERR_INVALID, "layer is NULL");
        if (nnz_x < 0 || (nnz_x > 0 && (!indices || !values)))
            throw_error(SILI_ERR_INVALID, "forward_sparse: bad CSR arguments");
        set_device(layer->L);
        forward_sparse(layer->L, ptrs, indices, values, nnz_x, batch, y, pick(layer->L, stream));
    });
}

int sili_backward_sparse(sili_layer *layer, const float *x, const int32_t *dy_ptrs, const int32_t *dy_indices,
                         const float *dy_values, int64_t nnz_dy, int64_t batch, float *dx, float learning_rate,
                         void *stream) {
    return guarded([&] {
        if (!layer) throw_error(SILI_ERR_INVALID, "layer is NULL");
        if (nnz_dy < 0 || (nnz_dy > 0 && (!dy_indices || !dy_values)))
            throw_error(SILI_ERR_INVALID, "backward_sparse: bad CSR arguments");
        set_device(layer->L);
        if (learning_rate != 0.0f) {
            // the reference binding's defaults (sili/cpu_backend.cpp:587-591)
            const TrainParams p{learning_rate, 0, 1, 0.999f, 1e-8f, 0.9f, 0.0f, 2.0f, 100.0f, 0.1f};
            backward_sparse_train(layer->L, x, dy_ptrs, dy_indices, dy_values, nnz_dy, batch, dx, p,
                                  pick(layer->L, stream));
            return;
        }
        backward_sparse(layer->L, x, dy_ptrs, dy_indices, dy_values, nnz_dy, batch, dx, pick(layer->L, stream));
    });
}

int sili_backward_sparse_train(sili_layer *layer, const float *x, const int32_t *dy_ptrs, const int32_t *dy_indices,
                               const float *dy_values, int64_t nnz_dy, int64_t batch, float *dx, float learning_rate,
                               int lr_per_row_nnz, int damp_by_importance, float beta2, float eps, void *stream) {
    return guarded([&] {
        if (!layer) throw_error(SILI_ERR_INVALID, "layer is NULL");
        if (nnz_dy < 0 || (nnz_dy > 0 && (!dy_indices || !dy_values)))
            throw_error(SILI_ERR_INVALID, "backward_sparse: bad CSR arguments");
        set_device(layer->L);
        hipStream_t st = pick(layer->L, stream);
        if (learning_rate == 0.0f) {
            backward_sparse(layer->L, x, dy_ptrs, dy_indices, dy_values, nnz_dy, batch, dx, st);
            return;
        }
        const TrainParams p{learning_rate, lr_per_row_nnz ? 1 : 0, damp_by_importance ? 1 : 0, beta2, eps,
                            0.9f, 0.0f, 2.0f, 100.0f, 0.1f};
        backward_sparse_train(layer->L, x, dy_ptrs, dy_indices, dy_values, nnz_dy, batch, dx, p, st);
    });
}

int sili_build_probes(sili_layer *layer, int64_t k, int per_row) {
    return guarded([&] {
        if (!layer) throw_error(SILI_ERR_INVALID, "layer is NULL");
        set_device(layer->L, true);
        build_probes(layer->L, k, per_row != 0);
    });
}

int sili_get_probes(sili_layer *layer, int64_t *n, int32_t *rows, int32_t *cols, float *scores, int64_t cap) {
    return guarded([&] {
        if (!layer || !n) throw_error(SILI_ERR_INVALID, "layer or n is NULL");
        const Layer &L = layer->L;
        *n = L.probe_nnz;
        for (int64_t i = 0; i < L.probe_nnz && i < cap; ++i) {
            if (rows) rows[i] = L.probe_r[(size_t)i];
            if (cols) cols[i] = L.probe_c[(size_t)i];
            if (scores) scores[i] = L.probe_v[(size_t)i];
        }
    });
}

int sili_synap_row_step(sili_layer *layer, int64_t *current_row, float importance_cutoff, int64_t max_row_weights,
                        int64_t max_prune_per_step, float importance_eps, int *did) {
    return guarded([&] {
        if (!layer || !current_row) throw_error(SILI_ERR_INVALID, "layer or current_row is NULL");
        if (*current_row < 0 || max_row_weights < 0 || max_prune_per_step < 0)
            throw_error(SILI_ERR_INVALID, "synap_row_step: negative row, max_row_weights or max_prune_per_step");
        set_device(layer->L, true);
        const bool r = synap_row_step(layer->L, *current_row, importance_cutoff, max_row_weights, max_prune_per_step,
                                      importance_eps);
        if (did) *did = r ? 1 : 0;
    });
}

int sili_synap_step(sili_layer *layer, float importance_cutoff, int64_t max_row_weights, int64_t max_prune_per_step,
                    float importance_eps, int *did) {
    if (!layer) return guarded([&] { throw_error(SILI_ERR_INVALID, "layer is NULL"); });
    return sili_synap_row_step(layer, &layer->L.synap_cursor, importance_cutoff, max_row_weights, max_prune_per_step,
                               importance_eps, did);
}

int sili_get_out_degree(sili_layer *layer, int32_t *out) {
    return guarded([&] {
        if (!layer || !out) throw_error(SILI_ERR_INVALID, "layer or out is NULL");
        set_device(layer->L, true);
        get_out_degree(layer->L, out);
    });
}

int sili_synapto_step(sili_layer *layer, float prune_frac, const int32_t *cand_rows, const int32_t *cand_cols,
                      const float *cand_vals, const float *cand_scores, int64_t n_cand, int default_imp_code,
                      int64_t *out_stats) {
    return guarded([&] {
        if (!layer) throw_error(SILI_ERR_INVALID, "layer is NULL");
        if (!(prune_frac >= 0.0f && prune_frac <= 1.0f)) throw_error(SILI_ERR_INVALID, "prune_frac must be in [0, 1]");
        if (n_cand < 0 || (n_cand > 0 && (!cand_rows || !cand_cols || !cand_vals)))
            throw_error(SILI_ERR_INVALID, "synapto_step: bad candidate arrays");
        if (default_imp_code < 0 || default_imp_code > 15) throw_error(SILI_ERR_INVALID, "default_imp_code must be a 4-bit code");
        set_device(layer->L);
        synapto_step(layer->L, prune_frac, cand_rows, cand_cols, cand_vals, cand_scores, n_cand, default_imp_code,
                     out_stats);
        layout_fit(layer->L);
        b4res_fit(layer->L);
    });
}

int sili_compact(sili_layer *layer) {
    return guarded([&] {
        if (!layer) throw_error(SILI_ERR_INVALID, "layer is NULL");
        set_device(layer->L);
        layout_compact(layer->L);
    });
}

int sili_expand_headroom(sili_layer *layer, float blank_fraction) {
    return guarded([&] {
        if (!layer) throw_error(SILI_ERR_INVALID, "layer is NULL");
        set_device(layer->L);
        layout_expand(layer->L, blank_fraction, -1);
    });
}

int sili_expand_headroom_to(sili_layer *layer, int64_t min_nnz_per_row, float blank_fraction) {
    return guarded([&] {
        if (!layer) throw_error(SILI_ERR_INVALID, "layer is NULL");
        // a negative count is a size_t beyond any budget to the reference
        if (min_nnz_per_row < 0) throw_error(SILI_ERR_NOMEM, "expand_headroom_to: min_nnz_per_row exceeds the budget");
        set_device(layer->L);
        layout_expand(layer->L, blank_fraction, min_nnz_per_row);
    });
}

int sili_equalize_to_capacity(sili_layer *layer, int64_t target_elems_per_row, int64_t target_bytes_per_row) {
    return guarded([&] {
        if (!layer) throw_error(SILI_ERR_INVALID, "layer is NULL");
        set_device(layer->L);
        layout_equalize_to_capacity(layer->L, target_elems_per_row, target_bytes_per_row);
    });
}

int sili_equalizer_step(sili_layer *layer) {
    return guarded([&] {
        if (!layer) throw_error(SILI_ERR_INVALID, "layer is NULL");
        set_device(layer->L);
        // the scattered store's step, then the block4 store's
        // (sili/cpu_backend.cpp:646-657)
        layout_equalizer_step(layer->L);
        b4res_equalize_step(layer->L);
    });
}

int sili_expand_block4_headroom(sili_layer *layer, float blank_fraction) {
    return guarded([&] {
        if (!layer) throw_error(SILI_ERR_INVALID, "layer is NULL");
        set_device(layer->L);
        b4res_expand(layer->L, blank_fraction, 16, b4_row_use(layer->L).ut);
    });
}

int sili_compact_block4(sili_layer *layer) {
    return guarded([&] {
        if (!layer) throw_error(SILI_ERR_INVALID, "layer is NULL");
        set_device(layer->L);
        b4res_expand(layer->L, 0.0f, 0, b4_row_use(layer->L).ut);
    });
}

int sili_export_block4_layout(sili_layer *layer, uint64_t *ia, uint64_t *ea, uint64_t *ta, uint64_t *ui,
                              uint64_t *ue, uint64_t *ut, uint64_t *out) {
    return guarded([&] {
        if (!layer) throw_error(SILI_ERR_INVALID, "layer is NULL");
        Layer &L = layer->L;
        set_device_read(L);
        const B4Use u = b4_row_use(L);
        const size_t rows = L.b4_ia.size();
        for (size_t r = 0; r < rows; ++r) {
            if (ia) ia[r] = L.b4_ia[r];
            if (ea) ea[r] = L.b4_ea[r];
            if (ta) ta[r] = L.b4_ta[r];
            if (ui) ui[r] = u.ui[r];
            if (ue) ue[r] = u.ue[r];
            if (ut) ut[r] = u.ut[r];
        }
        if (out) {
            uint64_t ctr[3];
            b4res_read_counters(L, ctr);
            out[0] = L.b4_dropped;
            out[1] = ctr[1];
            out[2] = ctr[2];
            out[3] = L.b4_idx_budget;
            out[4] = L.b4_tile_budget;
            out[5] = ctr[0];
        }
    });
}

int sili_export_layout(sili_layer *layer, uint64_t *byte_start, uint64_t *byte_end, uint64_t *elem_start,
                       uint64_t *elem_end) {
    return guarded([&] {
        if (!layer) throw_error(SILI_ERR_INVALID, "layer is NULL");
        set_device(layer->L);
        export_layout(layer->L, byte_start, byte_end, elem_start, elem_end);
    });
}

int sili_get_accumulators(sili_layer *layer, float *acc_in, float *acc_grad) {
    return guarded([&] {
        if (!layer) throw_error(SILI_ERR_INVALID, "layer is NULL");
        Layer &L = layer->L;
        set_device_read(L);
        SILI_HIP(hipStreamSynchronize(L.stream));
        if (acc_in) SILI_HIP(hipMemcpy(acc_in, L.acc_in.p, (size_t)L.n_in * 4, hipMemcpyDeviceToHost));
        if (acc_grad) SILI_HIP(hipMemcpy(acc_grad, L.acc_grad.p, (size_t)L.n_out * 4, hipMemcpyDeviceToHost));
    });
}

int sili_zero_accum(sili_layer *layer) {
    return guarded([&] {
        if (!layer) throw_error(SILI_ERR_INVALID, "layer is NULL");
        Layer &L = layer->L;
        set_device(L);
        fill(L.acc_in.p, L.n_in, 0.0f, L.stream);
        fill(L.acc_grad.p, L.n_out, 0.0f, L.stream);
    });
}

int sili_get_info(sili_layer *layer, sili_info *out) {
    return guarded([&] {
        if (!layer || !out) throw_error(SILI_ERR_INVALID, "NULL argument");
        Layer &L = layer->L;
        set_device_read(L);
        std::memset(out, 0, sizeof(*out));
        out->n_inputs = L.n_in;
        out->n_outputs = L.n_out;
        out->nnz_scattered = L.W.nnz;
        out->index_bytes = L.W.nbytes;
        out->n_tiles = L.B4.ntiles;
        out->block_index_bytes = L.B4.nbytes;
        out->n_segments = L.W.nseg;
        out->scale_rank = L.rank;
        out->has_nonfinite = L.has_nonfinite ? 1 : 0;
        out->stream_canonical = (L.W.stream1.valid || L.W.streamK.valid) ? 1 : 0;
        out->stream_shadow = (L.Wt.stream1.valid || L.Wt.streamK.valid) ? 1 : 0;
        out->split_combined = (L.W.part_cap > 0 ? 1 : 0) | (L.Wt.part_cap > 0 ? 2 : 0);
        out->short_rows_canonical = L.W.sh_valid ? L.W.n_sh : 0;
        out->short_rows_shadow = L.Wt.sh_valid ? L.Wt.n_sh : 0;
        if (L.B4.ntiles > 0) {
            std::vector<uint32_t> br, bc;
            export_block4_coords(L, br, bc);
            std::vector<uint8_t> t((size_t)L.B4.ntiles * 16);
            SILI_HIP(hipMemcpy(t.data(), L.B4.tiles.p, t.size(), hipMemcpyDeviceToHost));
            int64_t live = 0;
            for (size_t k = 0; k < br.size(); ++k)
                for (int s = 0; s < 16; ++s) {
                    const int64_t r = (int64_t)br[k] * 4 + (s & 3), c = (int64_t)bc[k] * 4 + (s >> 2);
                    live += (t[k * 16 + (size_t)s] != 0 && r < L.n_in && c < L.n_out) ? 1 : 0;
                }
            out->live_block4 = live;
        }
    });
}

int sili_export_scattered(sili_layer *layer, uint64_t *row_byte_start, uint64_t *row_elem_start, uint8_t *idx,
                          uint8_t *val) {
    return guarded([&] {
        if (!layer) throw_error(SILI_ERR_INVALID, "layer is NULL");
        Layer &L = layer->L;
        set_device_read(L);
        SILI_HIP(hipStreamSynchronize(L.stream));
        std::vector<uint32_t> tmp((size_t)L.n_in + 1);
        if (row_byte_start) {
            SILI_HIP(hipMemcpy(tmp.data(), L.W.byte_start.p, tmp.size() * 4, hipMemcpyDeviceToHost));
            for (size_t i = 0; i < tmp.size(); ++i) row_byte_start[i] = tmp[i];
        }
        if (row_elem_start) {
            SILI_HIP(hipMemcpy(tmp.data(), L.W.elem_start.p, tmp.size() * 4, hipMemcpyDeviceToHost));
            for (size_t i = 0; i < tmp.size(); ++i) row_elem_start[i] = tmp[i];
        }
        if (idx && L.W.nbytes) SILI_HIP(hipMemcpy(idx, L.W.idx.p, (size_t)L.W.nbytes, hipMemcpyDeviceToHost));
        if (val && L.W.nnz) SILI_HIP(hipMemcpy(val, L.W.val.p, (size_t)L.W.nnz, hipMemcpyDeviceToHost));
    });
}

namespace {
// FNV-1a over bytes copied from the device
uint64_t fnv(uint64_t h, const void *d_ptr, size_t bytes) {
    std::vector<uint8_t> v(bytes);
    if (bytes) SILI_HIP(hipMemcpy(v.data(), d_ptr, bytes, hipMemcpyDeviceToHost));
    for (uint8_t b : v) h = (h ^ b) * 0x100000001B3ull;
    return h;
}
uint64_t fnv_val(uint64_t h, int64_t x) {
    for (int k = 0; k < 8; ++k) h = (h ^ (uint8_t)(x >> (8 * k))) * 0x100000001B3ull;
    return h;
}
uint64_t digest_scatter(const DScatter &s) {
    uint64_t h = 0xCBF29CE484222325ull;
    for (int64_t x : {s.rows, s.cols, s.nnz, s.nbytes, s.nseg, s.n_empty_rows, (int64_t)s.has_split, s.n_split})
        h = fnv_val(h, x);
    h = fnv(h, s.byte_start.p, (size_t)(s.rows + 1) * 4);
    h = fnv(h, s.elem_start.p, (size_t)(s.rows + 1) * 4);
    h = fnv(h, s.idx.p, (size_t)s.nbytes);
    h = fnv(h, s.val.p, (size_t)s.nnz);
    h = fnv(h, s.seg.p, (size_t)s.nseg * sizeof(SegDesc));
    if (s.n_split) h = fnv(h, s.split_rows.p, (size_t)s.n_split * 4);
    return h;
}
uint64_t digest_b4(const DBlock4 &b, bool sparse) {
    uint64_t h = 0xCBF29CE484222325ull;
    for (int64_t x : {b.brows, b.bcols, b.ntiles, b.nbytes, b.nseg, (int64_t)b.has_split}) h = fnv_val(h, x);
    if (!b.byte_start.p) return h;
    h = fnv(h, b.byte_start.p, (size_t)(b.brows + 1) * 4);
    h = fnv(h, b.tile_start.p, (size_t)(b.brows + 1) * 4);
    h = fnv(h, b.idx.p, (size_t)b.nbytes);
    h = fnv(h, b.tiles.p, (size_t)b.ntiles * 16);
    h = fnv(h, b.seg.p, (size_t)b.nseg * sizeof(SegDesc));
    if (sparse) h = fnv(h, b.sparse.p, (size_t)b.ntiles);
    return h;
}
}  // namespace

int sili_debug_store_digest(sili_layer *layer, uint64_t *digest) {
    return guarded([&] {
        if (!layer || !digest) throw_error(SILI_ERR_INVALID, "layer or digest is NULL");
        Layer &L = layer->L;
        set_device_read(L);
        SILI_HIP(hipStreamSynchronize(L.stream));
        digest[0] = digest_scatter(L.W);
        digest[1] = digest_scatter(L.Wt);
        digest[2] = digest_b4(L.B4, true);
        digest[3] = digest_b4(L.B4t, false);
        const uint64_t h0 = 0xCBF29CE484222325ull;
        digest[4] = L.Wt_perm.p ? fnv(h0, L.Wt_perm.p, (size_t)L.Wt.nnz * 4) : 0;
        digest[5] = L.B4t_perm.p ? fnv(h0, L.B4t_perm.p, (size_t)L.B4t.ntiles * 4) : 0;
    });
}

int sili_export_block4(sili_layer *layer, int32_t *br, int32_t *bc, uint8_t *tiles, uint64_t *brow_byte_start,
                       uint64_t *brow_tile_start, uint8_t *bidx) {
    return guarded([&] {
        if (!layer) throw_error(SILI_ERR_INVALID, "layer is NULL");
        Layer &L = layer->L;
        set_device_read(L);
        SILI_HIP(hipStreamSynchronize(L.stream));
        if (br || bc) {
            std::vector<uint32_t> ubr, ubc;
            export_block4_coords(L, ubr, ubc);
            for (size_t i = 0; i < ubr.size(); ++i) {
                if (br) br[i] = (int32_t)ubr[i];
                if (bc) bc[i] = (int32_t)ubc[i];
            }
        }
        if (tiles && L.B4.ntiles)
            SILI_HIP(hipMemcpy(tiles, L.B4.tiles.p, (size_t)L.B4.ntiles * 16, hipMemcpyDeviceToHost));
        std::vector<uint32_t> tmp((size_t)L.B4.brows + 1);
        if (brow_byte_start) {
            SILI_HIP(hipMemcpy(tmp.data(), L.B4.byte_start.p, tmp.size() * 4, hipMemcpyDeviceToHost));
            for (size_t i = 0; i < tmp.size(); ++i) brow_byte_start[i] = tmp[i];
        }
        if (brow_tile_start) {
            SILI_HIP(hipMemcpy(tmp.data(), L.B4.tile_start.p, tmp.size() * 4, hipMemcpyDeviceToHost));
            for (size_t i = 0; i < tmp.size(); ++i) brow_tile_start[i] = tmp[i];
        }
        if (bidx && L.B4.nbytes) SILI_HIP(hipMemcpy(bidx, L.B4.idx.p, (size_t)L.B4.nbytes, hipMemcpyDeviceToHost));
    });
}

int sili_decode_scattered(sili_layer *layer, int32_t *cols, float *w_true) {
    return guarded([&] {
        if (!layer) throw_error(SILI_ERR_INVALID, "layer is NULL");
        Layer &L = layer->L;
        set_device_read(L);
        const size_t n = (size_t)L.W.nnz;
        if (n == 0) return;
        DevBuf<int32_t> dc;
        DevBuf<float> dw;
        dc.ensure(n);
        dw.ensure(n);
        launch_decode(L.W.plan(), canon_scales(L), dc.p, dw.p, nullptr, L.stream);
        SILI_HIP(hipStreamSynchronize(L.stream));
        if (cols) SILI_HIP(hipMemcpy(cols, dc.p, n * 4, hipMemcpyDeviceToHost));
        if (w_true) SILI_HIP(hipMemcpy(w_true, dw.p, n * 4, hipMemcpyDeviceToHost));
    });
}

int sili_export_absolute(sili_layer *layer, int32_t *ptrs, int32_t *indices, float *w, float *imp,
                         int64_t *n_out_entries) {
    return guarded([&] {
        if (!layer) throw_error(SILI_ERR_INVALID, "layer is NULL");
        Layer &L = layer->L;
        set_device_read(L);
        const size_t n = (size_t)L.W.nnz;
        std::vector<int32_t> cols(n);
        std::vector<uint8_t> val(n);
        std::vector<uint32_t> elem((size_t)L.n_in + 1);
        if (n) {
            DevBuf<int32_t> dc;
            dc.ensure(n);
            const ScaleView none{nullptr, nullptr, 1};
            launch_decode(L.W.plan(), none, dc.p, nullptr, nullptr, L.stream);
            SILI_HIP(hipStreamSynchronize(L.stream));
            SILI_HIP(hipMemcpy(cols.data(), dc.p, n * 4, hipMemcpyDeviceToHost));
            SILI_HIP(hipMemcpy(val.data(), L.W.val.p, n, hipMemcpyDeviceToHost));
        }
        SILI_HIP(hipMemcpy(elem.data(), L.W.elem_start.p, elem.size() * 4, hipMemcpyDeviceToHost));
        std::vector<uint32_t> br, bc;
        std::vector<uint8_t> tiles;
        export_block4_coords(L, br, bc);
        tiles.resize(br.size() * 16);
        if (!br.empty()) SILI_HIP(hipMemcpy(tiles.data(), L.B4.tiles.p, tiles.size(), hipMemcpyDeviceToHost));
        // tiles of each block row, in storage (bc ascending) order
        std::vector<size_t> tb((size_t)((L.n_in + 3) / 4) + 1, 0);
        for (uint32_t r : br) tb[(size_t)r + 1]++;
        for (size_t i = 1; i < tb.size(); ++i) tb[i] += tb[i - 1];
        struct E { int32_t c; float w, imp; };
        std::vector<E> row;
        int64_t flat = 0;
        if (ptrs) ptrs[0] = 0;
        for (int64_t r = 0; r < L.n_in; ++r) {
            row.clear();
            for (uint32_t e = elem[(size_t)r]; e < elem[(size_t)r + 1]; ++e)
                row.push_back({cols[e], fp4_decode(val[e] >> 4), fp4_decode(val[e] & 0xFu)});
            const int64_t b = r / 4, li = r % 4;
            for (size_t k = tb[(size_t)b]; k < tb[(size_t)b + 1]; ++k)
                for (int lj = 0; lj < 4; ++lj) {
                    const uint8_t byte = tiles[k * 16 + (size_t)(lj * 4 + li)];
                    const int64_t c = (int64_t)bc[k] * 4 + lj;
                    if (byte == 0 || c >= L.n_out) continue;
                    row.push_back({(int32_t)c, fp4_decode(byte & 0xFu), fp4_decode(byte >> 4)});
                }
            std::stable_sort(row.begin(), row.end(), [](const E &a, const E &b2) { return a.c < b2.c; });
            for (const E &e : row) {
                if (indices) indices[flat] = e.c;
                if (w) w[flat] = e.w;
                if (imp) imp[flat] = e.imp;
                ++flat;
            }
            if (ptrs) ptrs[r + 1] = (int32_t)flat;
        }
        if (n_out_entries) *n_out_entries = flat;
    });
}

int sili_profile_enable(sili_layer *layer, int enable) {
    return guarded([&] {
        if (!layer) throw_error(SILI_ERR_INVALID, "layer is NULL");
        Profiler &P = layer->L.prof;
        set_device(layer->L);
        SILI_HIP(hipStreamSynchronize(layer->L.stream));
        for (auto &r : P.recs) { P.pool.push_back(r.a); P.pool.push_back(r.b); }
        P.recs.clear();
        P.enabled = enable != 0;
    });
}

int sili_profile_read(sili_layer *layer, sili_prof_entry *out, int max_entries, int *n_entries) {
    return guarded([&] {
        if (!layer) throw_error(SILI_ERR_INVALID, "layer is NULL");
        Profiler &P = layer->L.prof;
        set_device(layer->L);
        std::vector<sili_prof_entry> agg;
        for (auto &r : P.recs) {
            SILI_HIP(hipEventSynchronize(r.b));
            float ms = 0.0f;
            SILI_HIP(hipEventElapsedTime(&ms, r.a, r.b));
            sili_prof_entry *e = nullptr;
            for (auto &a : agg)
                if (r.name == a.name) e = &a;
            if (!e) {
                agg.push_back(sili_prof_entry{});
                e = &agg.back();
                std::strncpy(e->name, r.name.c_str(), sizeof(e->name) - 1);
                e->min_ms = 1e30;
            }
            e->count += 1;
            e->total_ms += ms;
            e->min_ms = std::min(e->min_ms, (double)ms);
            e->max_ms = std::max(e->max_ms, (double)ms);
            P.pool.push_back(r.a);
            P.pool.push_back(r.b);
        }
        P.recs.clear();
        if (n_entries) *n_entries = (int)agg.size();
        for (int i = 0; out && i < (int)agg.size() && i < max_entries; ++i) out[i] = agg[(size_t)i];
    });
}

int sili_export_block4_packed(sili_layer *layer, uint8_t *tile_is_sparse, uint8_t *tile_data,
                              uint64_t *tile_byte_start, int64_t *nbytes) {
    return guarded([&] {
        if (!layer || !nbytes) throw_error(SILI_ERR_INVALID, "NULL argument");
        Layer &L = layer->L;
        set_device(L);
        const PackedTiles pk = export_tiles_packed(L);
        *nbytes = (int64_t)pk.bytes.size();
        if (tile_is_sparse && !pk.flags.empty()) std::memcpy(tile_is_sparse, pk.flags.data(), pk.flags.size());
        if (tile_data && !pk.bytes.empty()) std::memcpy(tile_data, pk.bytes.data(), pk.bytes.size());
        if (tile_byte_start)
            std::memcpy(tile_byte_start, pk.row_start.data(), pk.row_start.size() * sizeof(uint64_t));
    });
}

int sili_block4_view(sili_layer *layer, sili_block4_stats *out) {
    return guarded([&] {
        if (!layer || !out) throw_error(SILI_ERR_INVALID, "NULL argument");
        Layer &L = layer->L;
        set_device(L);
        const PackedTiles pk = export_tiles_packed(L);
        out->tiles = L.B4.ntiles;
        out->synapses = pk.live;
        out->switch_point = L.switch_point;
        out->used_bytes = (int64_t)pk.bytes.size();
        uint64_t alloc = 0, ctr[3];
        for (uint64_t v : L.b4_ta) alloc += v;
        b4res_read_counters(L, ctr);
        out->alloc_bytes = (int64_t)alloc;
        out->dropped_growth_events = (int64_t)L.b4_dropped;
        out->row_merge_overflow_events = (int64_t)ctr[1];
        out->row_merge_overflow_bytes_dropped = (int64_t)ctr[2];
    });
}

int sili_set_switch_point(sili_layer *layer, uint32_t switch_point) {
    return guarded([&] {
        if (!layer) throw_error(SILI_ERR_INVALID, "layer is NULL");
        if (switch_point > 10)
            throw_error(SILI_ERR_INVALID, "switch_point must be <= 10 (a sparse-packed tile of more live "
                                          "slots is longer than a dense one, block4.hpp:332-340)");
        layer->L.switch_point = switch_point;
    });
}

int sili_build_for_index(sili_layer *layer, int group_size) {
    return guarded([&] {
        if (!layer) throw_error(SILI_ERR_INVALID, "layer is NULL");
        set_device(layer->L);
        ProfCtx pc(layer->L, "index");
        build_for_index(layer->L, group_size);
    });
}

int sili_export_for_index(sili_layer *layer, uint64_t *row_byte_start, uint8_t *bytes, int64_t *nbytes) {
    return guarded([&] {
        if (!layer || !nbytes) throw_error(SILI_ERR_INVALID, "NULL argument");
        Layer &L = layer->L;
        set_device(L);
        const DFor &F = L.W.fidx;
        if (!F.valid) throw_error(SILI_ERR_INVALID, "export_for_index: build the FOR index first");
        *nbytes = F.nbytes;
        if (row_byte_start) {
            std::vector<uint32_t> rg((size_t)L.n_in + 1), gp((size_t)F.ngroups + 1);
            SILI_HIP(hipMemcpyAsync(rg.data(), F.row_group.p, rg.size() * 4, hipMemcpyDeviceToHost, L.stream));
            SILI_HIP(hipMemcpyAsync(gp.data(), F.group_pos.p, gp.size() * 4, hipMemcpyDeviceToHost, L.stream));
            SILI_HIP(hipStreamSynchronize(L.stream));
            for (size_t r = 0; r < rg.size(); ++r) row_byte_start[r] = gp[rg[r]];
        }
        if (bytes && F.nbytes) {
            SILI_HIP(hipMemcpyAsync(bytes, F.bytes.p, (size_t)F.nbytes, hipMemcpyDeviceToHost, L.stream));
            SILI_HIP(hipStreamSynchronize(L.stream));
        }
    });
}

int sili_decode_columns(sili_layer *layer, int32_t *cols, int use_for_index, void *stream) {
    return guarded([&] {
        if (!layer) throw_error(SILI_ERR_INVALID, "layer is NULL");
        set_device(layer->L);
        if (!cols && layer->L.W.nnz > 0) throw_error(SILI_ERR_INVALID, "cols is NULL");
        ProfCtx pc(layer->L, "index");
        if (use_for_index < 0 || use_for_index > 2) throw_error(SILI_ERR_INVALID, "use_for_index must be 0, 1 or 2");
        decode_columns(layer->L, cols, use_for_index, pick(layer->L, stream));
    });
}

int sili_fp4_quantize(const float *x, int64_t n, uint8_t *codes, void *stream) {
    return guarded([&] {
        if (n < 0) throw_error(SILI_ERR_INVALID, "fp4_quantize: negative length");
        if (n == 0) return;
        if (!x || !codes) throw_error(SILI_ERR_INVALID, "fp4_quantize: NULL buffer");
        hipStream_t st = reinterpret_cast<hipStream_t>(stream);
        launch(k_fp4_codes, dim3(nblk(n)), dim3(TPB), 0, st, x, n, codes);
        SILI_HIP(hipGetLastError());
        SILI_HIP(hipStreamSynchronize(st));
    });
}

int sili_dense_to_csr(const float *x, int64_t rows, int64_t cols, float threshold, int32_t *ptrs, int32_t *indices,
                      float *values, int64_t capacity, int64_t *nnz, void *stream) {
    return guarded([&] {
        if (!nnz) throw_error(SILI_ERR_INVALID, "dense_to_csr: nnz is NULL");
        dense_to_csr_device(x, rows, cols, threshold, ptrs, indices, values, capacity, nnz,
                            reinterpret_cast<hipStream_t>(stream));
    });
}

int sili_dense_to_top_k_csr(const float *x, int64_t rows, int64_t cols, int64_t k, int32_t *ptrs, int32_t *indices,
                            float *values, int64_t *nnz, void *stream) {
    return guarded([&] {
        if (!nnz) throw_error(SILI_ERR_INVALID, "dense_to_top_k_csr: nnz is NULL");
        dense_to_top_k_csr_device(x, rows, cols, k, ptrs, indices, values, nnz, reinterpret_cast<hipStream_t>(stream));
    });
}

int sili_buffer_alloc(int device, size_t bytes, void **out) {
    return guarded([&] {
        if (!out) throw_error(SILI_ERR_INVALID, "NULL argument");
        SILI_HIP(hipSetDevice(device));
        SILI_HIP(hipMalloc(out, bytes ? bytes : 1));
    });
}
int sili_buffer_free(int device, void *ptr) {
    return guarded([&] {
        SILI_HIP(hipSetDevice(device));
        if (ptr) SILI_HIP(hipFree(ptr));
    });
}
int sili_buffer_copy(int device, void *dst, const void *src, size_t bytes) {
    return guarded([&] {
        SILI_HIP(hipSetDevice(device));
        if (bytes) SILI_HIP(hipMemcpy(dst, src, bytes, hipMemcpyDefault));
    });
}

int sili_device_alloc(sili_layer *layer, size_t bytes, void **out) {
    return guarded([&] {
        if (!layer || !out) throw_error(SILI_ERR_INVALID, "NULL argument");
        set_device(layer->L);
        SILI_HIP(hipMalloc(out, bytes ? bytes : 1));
    });
}
int sili_device_free(sili_layer *layer, void *ptr) {
    return guarded([&] {
        if (!layer) throw_error(SILI_ERR_INVALID, "NULL argument");
        set_device(layer->L);
        if (ptr) SILI_HIP(hipFree(ptr));
    });
}
int sili_memcpy_h2d(sili_layer *layer, void *dst, const void *src, size_t bytes) {
    return guarded([&] {
        if (!layer) throw_error(SILI_ERR_INVALID, "NULL argument");
        set_device(layer->L);
        SILI_HIP(hipStreamSynchronize(layer->L.stream));
        if (bytes) SILI_HIP(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
    });
}
int sili_memcpy_d2h(sili_layer *layer, void *dst, const void *src, size_t bytes) {
    return guarded([&] {
        if (!layer) throw_error(SILI_ERR_INVALID, "NULL argument");
        set_device(layer->L);
        SILI_HIP(hipStreamSynchronize(layer->L.stream));
        if (bytes) SILI_HIP(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
    });
}
int sili_host_alloc(size_t bytes, void **out) {
    return guarded([&] {
        if (!out) throw_error(SILI_ERR_INVALID, "NULL argument");
        *out = nullptr;
        if (hipHostMalloc(out, bytes ? bytes : 4, hipHostMallocDefault) != hipSuccess || !*out) {
            (void)hipGetLastError();
            throw_error(SILI_ERR_NOMEM, "sili_host_alloc: hipHostMalloc failed");
        }
    });
}
int sili_host_free(void *ptr) {
    return guarded([&] {
        if (ptr) SILI_HIP(hipHostFree(ptr));
    });
}
int sili_memcpy_h2d_ordered(sili_layer *layer, void *dst, const void *src, size_t bytes) {
    return guarded([&] {
        if (!layer) throw_error(SILI_ERR_INVALID, "NULL argument");
        set_device(layer->L);
        if (!bytes) return;
        if (host_locked(src)) kernel_copy(dst, src, bytes, layer->L.stream);
        else SILI_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, layer->L.stream));
    });
}
int sili_memcpy_d2h_ordered(sili_layer *layer, void *dst, const void *src, size_t bytes) {
    return guarded([&] {
        if (!layer) throw_error(SILI_ERR_INVALID, "NULL argument");
        set_device(layer->L);
        if (bytes && host_locked(dst)) kernel_copy(dst, src, bytes, layer->L.stream);
        else if (bytes) SILI_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, layer->L.stream));
        SILI_HIP(hipStreamSynchronize(layer->L.stream));
    });
}
int sili_memset_device(sili_layer *layer, void *dst, int value, size_t bytes) {
    return guarded([&] {
        if (!layer) throw_error(SILI_ERR_INVALID, "NULL argument");
        set_device(layer->L);
        if (bytes) SILI_HIP(hipMemsetAsync(dst, value, bytes, layer->L.stream));
        SILI_HIP(hipStreamSynchronize(layer->L.stream));
    });
}

}  // extern "C"
