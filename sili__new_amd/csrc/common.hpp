// common.hpp -- shared definitions of the gfx950 FP4 delta-CSR layer library.
//
// Device storage per layer (all compact, no per-row headroom):
//   scattered store, canonical (rows = input neurons) and shadow (rows =
//   output neurons, the transpose rebuilt on the device after every
//   structural change):
//     byte_start[rows+1], elem_start[rows+1]  uint32
//     idx[]   ULEB128 column deltas, first delta from 0 on every row
//     val[]   one byte per synapse, (w_code<<4)|imp_code
//     seg[]   decode work items (see SegDesc)
//   block4 store, canonical (block rows over inputs) and shadow (block rows
//   over outputs, tile bytes 4x4-transposed):
//     byte_start/tile_start[brows+1] uint32, idx[] ULEB128 block-column
//     deltas, tiles[16*n] (slot lj*4+li, byte (imp<<4)|w), seg[].
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>

#include <cstddef>
#include <cstdint>
#include <cstdlib>
#include <string>
#include <tuple>

namespace sili {

// Integer tuning knob from the environment.
inline int env_int(const char *name, int dflt) {
    const char *e = std::getenv(name);
    return e ? std::atoi(e) : dflt;
}

// ---- error plumbing (host) ------------------------------------------------
struct Error {
    int code;
    std::string msg;
};
[[noreturn]] void throw_error(int code, const std::string &msg);
void hip_check(hipError_t e, const char *what);
#define SILI_HIP(expr) ::sili::hip_check((expr), #expr)

// ---- measurement ------------------------------------------------------------
// When a layer's profiler is enabled, every kernel launched through launch()
// inside a ProfScope carries a hipEvent pair that the runtime stamps with that
// dispatch's own begin and end (hipExtLaunchKernel), accounted under
// "<op>:<kernel>" (sili_profile_read).  The times are those of the kernel
// alone, without the queue gaps a separate hipEventRecord marker would add.
// Disabled: launch() is a plain hipLaunchKernelGGL.
struct ProfOp {              // names the entry point for the launches below it
    explicit ProfOp(const char *op);
    ~ProfOp();
    const char *prev;
};
struct ProfScope {           // names the kernel(s) launched while it lives
    ProfScope(const char *kernel, hipStream_t st);
    ~ProfScope();
    const char *prev;
};
// Events for the next launch when it is profiled (false: not profiled).
bool prof_next(hipEvent_t *start, hipEvent_t *stop);

template <typename... KArgs, typename... Args>
void launch(void (*kernel)(KArgs...), dim3 grid, dim3 block, uint32_t shmem, hipStream_t st,
            Args... args) {
    static_assert(sizeof...(KArgs) == sizeof...(Args), "kernel argument count");
    hipEvent_t a, b;
    if (!prof_next(&a, &b)) {
        hipLaunchKernelGGL(kernel, grid, block, shmem, st, static_cast<KArgs>(args)...);
        return;
    }
    std::tuple<KArgs...> tup{static_cast<KArgs>(args)...};
    std::apply([&](auto &...e) {
        void *ptrs[] = {static_cast<void *>(&e)...};
        SILI_HIP(hipExtLaunchKernel(reinterpret_cast<const void *>(kernel), grid, block, ptrs, shmem,
                                    st, a, b, 0));
    }, tup);
}

// ---- decode work item ------------------------------------------------------
// One contiguous run of a row's entries, starting at a varint boundary with a
// known running column (the column of the entry before it, 0 at row start),
// spanning at most SEG_BYTES_MAX index bytes.  Rows longer than that are
// split; `split` marks every segment of such a row (their partial sums are
// combined with atomics).
struct alignas(32) SegDesc {
    uint32_t row;
    uint32_t byte_begin;
    uint32_t byte_end;
    uint32_t elem_begin;
    uint32_t base_col;
    uint32_t split;   // SEG_SPLIT | SEG_FIRST
    uint32_t elem_end;
    uint32_t pad1;
};
// Index bytes per segment are capped (the kernels stage a whole segment in
// LDS).  448: a block of 4 float4-gather waves then needs 20,384 bytes of
// LDS (staged bytes + the entry table), so 8 blocks share a CU's 160 KiB.
constexpr uint32_t SEG_BYTES_MAX = 448;

constexpr uint32_t SEG_SPLIT = 1u;  // the row has several segments (combine with atomics)
constexpr uint32_t SEG_FIRST = 2u;  // first segment of its row

// ---- stream window ---------------------------------------------------------
// The stream kernels read a padded copy of a scattered store (see DStream in
// layer.hpp) cut into windows of WIN_BYTES = 64 lanes x 16 bytes.  Per window:
//   carry : shifted column (col + 1) of the last entry ending before the
//           window in the row holding the window's first byte (0 if none)
//   rs_lo : first non-empty row (index into the store's list of non-empty
//           rows) whose first byte is at or after the window start
//   mask  : bit l set when a non-empty row starts at byte 16 l of the window
//           (rows start 16-byte aligned; popcount(mask) rows start here, the
//           next window's rs_lo is rs_lo + popcount(mask), and the row holding
//           the first byte is list entry rs_lo - 1 unless bit 0 is set)
// A sentinel follows the last window: {0, number of non-empty rows, 0, 0}.
constexpr uint32_t WIN_BYTES = 1024;
struct alignas(16) WinDesc {
    uint32_t carry, rs_lo, mask_lo, mask_hi;
};

// ---- FP4 E2M1 codec (device + host) -----------------------------------------
// Code c = s<<3 | e<<1 | m, bias 1; code 8 is NaN (0x7FC00000), not -0
// (reference fp4quant.hpp:16-33,68-84).
__host__ __device__ __forceinline__ float fp4_decode(uint32_t code) {
    const uint32_t s = (code >> 3) & 1u, e = (code >> 1) & 3u, m = code & 1u;
    uint32_t bits;
    if (e == 0) bits = m ? (0x3F000000u | (s << 31)) : (s ? 0x7FC00000u : 0u);
    else bits = (s << 31) | ((e + 126u) << 23) | (m << 22);
    return __builtin_bit_cast(float, bits);
}

// Nearest code; ties away from zero (rounding carry), saturate at 6, NaN -> 0,
// |v| < 0.25 -> 0, never the NaN slot (reference fp4quant.hpp:86-121).
__host__ __device__ __forceinline__ uint32_t fp4_encode(float v) {
    const uint32_t bits = __builtin_bit_cast(uint32_t, v);
    const uint32_t a = bits & 0x7FFFFFFFu;
    uint32_t mag;
    if (a > 0x7F800000u) return 0;
    if (a < 0x3E800000u) mag = 0;
    else if (a < 0x3F400000u) mag = 1;
    else if (a < 0x3F800000u) mag = 2;
    else {
        uint32_t r = a + (1u << 21);
        r = r > 0x40C00000u ? 0x40C00000u : r;
        mag = ((((r >> 23) & 0xFFu) - 126u) << 1) | ((r >> 22) & 1u);
    }
    if (mag == 0) return 0;
    return ((bits >> 31) << 3) | mag;
}

// ULEB128 length of v (1..5 bytes).
__host__ __device__ __forceinline__ uint32_t uleb_len(uint32_t v) {
    return v < (1u << 7) ? 1u : v < (1u << 14) ? 2u : v < (1u << 21) ? 3u : v < (1u << 28) ? 4u : 5u;
}

// A block4 tile's stored length (block4_stored_tile_len, block4.hpp:340-345):
// sparse-packed [count][ceil(live/2) position bytes][live values], or the 16
// dense bytes.
__host__ __device__ __forceinline__ uint32_t tile_len(bool sparse, uint32_t live) {
    return sparse ? 1u + (live + 1u) / 2u + live : 16u;
}

// ---- host-side launchers (kernels.hip / build.hip / synapto.hip) -----------
struct ScaleView {
    const float *row;   // scale indexed by the gather row   [rows*rank]
    const float *ent;   // scale indexed by the entry index  [cols*rank], NULL = all ones (rank 1)
    int rank;
};

enum SkipMode : int { SKIP_NONE = 0, SKIP_ZERO = 1, SKIP_POSZERO = 2 };

struct GatherPlan {      // one orientation of the scattered store
    const SegDesc *seg;
    int64_t nseg;
    const uint8_t *idx;
    const uint8_t *val;
    int64_t rows, cols;
    bool has_split;
    const uint32_t *split_rows;  // rows spanning several work items (n_split of them)
    int64_t n_split;
    // split rows combined without float atomics (the float4 gather): each
    // work item of a split row leaves its partial sums in part[si * nb ...],
    // the last one of its row to finish (arrivals counted in split_cnt, by
    // entries against elem_start) adds the row's items in order; part ==
    // nullptr: combined by atomics.  part_cap: floats part holds.
    const uint32_t *elem_start = nullptr;
    uint32_t *split_cnt = nullptr;
    float *part = nullptr;
    int64_t part_cap = 0;
    // short rows packed several to a wave by the float4 gather (set only by
    // gather_plan; nullptr: every work item takes a wave): sh_seg lists the
    // work items that are whole rows of at most SHORT_ROW_BYTES index bytes,
    // lg_seg the others, both in store order
    const SegDesc *sh_seg = nullptr;
    int64_t n_sh = 0;
    const SegDesc *lg_seg = nullptr;
    int64_t n_lg = 0;
};

// Short rows: a wave of the float4 gather takes up to SHORT_R_MAX of them,
// their index bytes staged back to back (SHORT_R_MAX * SHORT_ROW_BYTES <=
// SEG_BYTES_MAX) and their results held in the wave's entry table
// (SHORT_R_MAX * batch floats, batch <= SHORT_MAX_BATCH).
constexpr uint32_t SHORT_R_MAX = 16;
constexpr uint32_t SHORT_ROW_BYTES = 28;
constexpr int64_t SHORT_MAX_BATCH = 64;

struct Block4Plan {
    const SegDesc *seg;
    int64_t nseg;
    const uint8_t *idx;
    const uint8_t *tiles;
    int64_t rows, cols;  // element rows / cols of this orientation
    bool has_split;
};

// out[b*out_ld + row] for b < nb: scattered gather (stores; atomics for split
// rows -- then the caller has zeroed out).  in is feature-major in[c*in_ld + b].
// accumulate: add to out (batches with nb % 4 == 0 and aligned feature-major
// input only; used by the column-block passes).
void launch_gather(const GatherPlan &p, const ScaleView &sc, const float *in, int64_t in_ld,
                   float *out, int64_t out_ld, int64_t nb, int skip, hipStream_t st, bool accumulate = false);
// Block4 contribution, added into out.
void launch_gather_b4(const Block4Plan &p, const ScaleView &sc, const float *in, int64_t in_ld,
                      float *out, int64_t out_ld, int64_t nb, int skip, hipStream_t st);
// gw[e] = sum_b xT[row*B+b] * gT[col*B+b] over the canonical store; when
// acc_in != NULL also acc_in[row] += sum_b |xT[row*B+b]| for every row.
// Fused grad-input gather + sampled grad-W over the canonical store (one
// decode, one gT load per synapse).  Returns false, launching nothing, when
// the operands do not fit the fused kernel (B % 4, B > 512, alignment).
bool launch_bwd_fused(const GatherPlan &p, const ScaleView &sc, const float *gT, const float *xT,
                      int64_t B, float *dx, int64_t dx_ld, float *gw, float *acc_in, hipStream_t st);
void launch_sddmm(const GatherPlan &p, const float *xT, const float *gT, int64_t B, float *gw,
                  float *acc_in, hipStream_t st);
// acc[j] += sum_b |xT[j*B+b]| (feature-major input).
void launch_rowabs(const float *xT, int64_t B, int64_t n, float *acc, hipStream_t st);
// Independent small tasks in one launch (k_prep): a transpose [B, n] -> [n, B]
// with optional sum |.| per column into acc (B % 4 == 0, n % 4 == 0,
// 16-byte aligned src and dst), sum |src[b, j]| over the batch into acc[j]
// (n % 4 == 0, aligned src and acc), sum over a feature-major row into acc,
// a float4 fill of n float4 with v, zeroing out[b * ld + rows[r]] for
// r < n split rows and b < B.
enum : int { PREP_TRANSPOSE = 0, PREP_COLABS = 1, PREP_ROWABS = 2, PREP_FILL4 = 3, PREP_ZERO_LIST = 4 };
struct PrepTask {
    int kind;
    uint32_t first;  // set by launch_prep
    const float *src;
    float *dst, *acc;
    int64_t B, n, ld;
    const uint32_t *rows;
    float v;
};
constexpr int PREP_MAX = 4;
struct PrepArgs {
    PrepTask t[PREP_MAX];
    int nt;
};
void launch_prep(const PrepTask *tasks, int nt, hipStream_t st);
// A block4 store's tiles by column range: tcol[t] = the block column of
// tile t; run (x, br) = tiles [start[x*brows + br], start[(x+1)*brows + br]).
struct B4Ranges {
    const uint32_t *tcol, *start;
    int64_t K, brows;
};
// gw[16t + lj*4+li] = sum_b xT[4br+li, b] * gT[4bc+lj, b] for every tile t;
// rng (optional, K >= 1 built): by column range, range x on XCD x.
void launch_sddmm_b4(const Block4Plan &p, const B4Ranges *rng, const float *xT,
                     const float *gT, int64_t B, float *gw, hipStream_t st);
// [B, n] -> [n, B]; when acc != NULL also acc[j] += sum_b |src[b, j]|.
void launch_transpose(const float *src, int64_t B, int64_t n, float *dst, float *acc,
                      hipStream_t st);
// acc[j] += sum_b |src[b, j]| (no transpose).
void launch_colabs(const float *src, int64_t B, int64_t n, float *acc, hipStream_t st);
// CSR (ptrs[B+1], idx, vals) -> dense feature-major dst[idx*B + b] (dst pre-zeroed).
// When mark_explicit, explicit zero values are written as -0.0 so that
// SKIP_POSZERO can tell them from absent entries.
// nnz_hint: the number of stored entries (ptrs[batch]) when known on the
// host -- one thread per entry; 0: one block per batch row.
// The whole feature-major [n, B] array from CSR activations whose indices
// ascend within each batch row (zeros where absent; explicit zeros -0.0 when
// mark_explicit; acc_abs[j] += |v| when given): no separate zero fill.
void launch_densify_full(const int32_t *ptrs, const int32_t *idx, const float *vals, int64_t B, int64_t n,
                         float *dst, float *acc_abs, bool mark_explicit, int64_t nnz, hipStream_t st);
// Zero out[b, row] of the rows split over several work items of `p`.
void launch_zero_split_rows(const GatherPlan &p, float *out, int64_t out_ld, int64_t nb, hipStream_t st);

// Device decode of a scattered store: cols[e], w[e] = fl32(dec * S(row, col)).
void launch_decode(const GatherPlan &p, const ScaleView &sc, int32_t *cols, float *w,
                   uint32_t *rows_out, hipStream_t st);
// Block4 decode: for every tile, its block row, block column and storage index.
void launch_decode_b4(const Block4Plan &p, uint32_t *tile_br, uint32_t *tile_bc,
                      hipStream_t st);

}  // namespace sili
