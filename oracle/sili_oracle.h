/*
 * sili_oracle.h -- CPU restatement of the reference's FP4 delta-CSR sparse
 * layer arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (sili__new_amd/, the
 * C-ABI library, bench.py's GPU leg) may link, load or call this code.  It
 * is the checker for the HIP path (tests/, __graft_entry__.smoke()) and the
 * timed CPU baseline in bench.py's cpu_baseline leg.
 *
 * Every function cites the reference file:line it restates (paths relative
 * to the SimLeek/sili__new tree).  Pinning status of each function is listed
 * in oracle/README.md.
 *
 * Layout conventions (reference semantics):
 *   - rows of the weight matrix are INPUT neurons (linear_disldo.hpp:63-65);
 *   - activations are [batch, n] row-major fp32 (linear_disldo.hpp:41-44);
 *   - scattered value byte = (w_code << 4) | imp_code (fp4quant.hpp:280-383);
 *   - block4 slot byte     = (imp_code << 4) | w_code, slot = lj*4 + li
 *     (block4.hpp:300-312);
 *   - column indices are ULEB128 deltas, first delta from 0 on every row
 *     (delta_csr_memory.hpp:45-52,78-90).
 */
#ifndef SILI_ORACLE_H
#define SILI_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Flat, compact (headroom-free) view of one layer. */
typedef struct {
    int64_t n_in, n_out;
    int32_t rank;                   /* scale rank, 1..4 */
    /* scattered delta-CSR */
    const uint64_t *row_byte_start; /* [n_in+1] */
    const uint64_t *row_elem_start; /* [n_in+1] */
    const uint8_t  *idx;            /* ULEB128 column deltas */
    const uint8_t  *val;            /* (w<<4)|imp, one byte per synapse */
    /* block4 store (dense 16-byte tiles) */
    int64_t n_tiles;
    const uint64_t *brow_byte_start; /* [ceil(n_in/4)+1] or NULL when n_tiles==0 */
    const uint64_t *brow_tile_start; /* [ceil(n_in/4)+1] */
    const uint8_t  *bidx;            /* ULEB128 block-column deltas */
    const uint8_t  *tiles;           /* 16 bytes per tile */
    /* scales, row-major per component: vs[r*rank+k], os[c*rank+k] */
    const float *value_scale;       /* [n_in*rank] */
    const float *output_scale;      /* [n_out*rank] */
} OracleLayer;

/* ---- codecs ---- */
float   oracle_fp4_decode(uint8_t code);
uint8_t oracle_fp4_encode(float v);
void    oracle_fp4_encode_array(const float *v, int64_t n, uint8_t *out);
size_t  oracle_uleb_encode(uint32_t v, uint8_t *out);
uint32_t oracle_uleb_decode(const uint8_t *buf, uint64_t *pos);

/* ---- structure ---- */
/* Byte count of the compact ULEB stream for an absolute CSR. */
int64_t oracle_csr_index_bytes(int64_t rows, const int32_t *ptrs, const int32_t *idx);
/* Absolute CSR -> compact delta-CSR.  w/imp are quantized with fp4_encode. */
int oracle_csr_encode(int64_t rows, const int32_t *ptrs, const int32_t *idx,
                      const float *w, const float *imp,
                      uint64_t *row_byte_start, uint64_t *row_elem_start,
                      uint8_t *idx_out, uint8_t *val_out);
/* Same, from pre-built value bytes (no quantization). */
int oracle_csr_encode_bytes(int64_t rows, const int32_t *ptrs, const int32_t *idx,
                            const uint8_t *bytes,
                            uint64_t *row_byte_start, uint64_t *row_elem_start,
                            uint8_t *idx_out, uint8_t *val_out);
/* Compact delta-CSR -> absolute columns (int32) in elem order. */
int oracle_csr_decode(int64_t rows, const uint64_t *row_byte_start,
                      const uint64_t *row_elem_start, const uint8_t *idx,
                      int32_t *cols_out);

/* Combined (scattered + block4 live slots) absolute CSR, per row sorted by
 * column, decoded values (FP4_TABLE) -- delta_csr_memory.hpp:127-213.
 * Returns total entries; call with NULL outputs to size. */
int64_t oracle_combined_to_absolute(const OracleLayer *L, int32_t *ptrs,
                                    int32_t *idx, float *w, float *imp);

/* Dense true-weight matrix W[r*n_out+c] = dec(code)*S(r,c) (scattered
 * association dec*(vs*os)); 0 where nothing is stored. */
void oracle_dense_weights(const OracleLayer *L, float *W);

/* ---- compute (lr = 0 semantics; outputs ACCUMULATE, caller zeroes) ----
 * absmode != 0 replaces every weight and activation by its magnitude, giving
 * the per-output sum of |terms| used by the condition-aware tolerance. */
void oracle_forward_dense(const OracleLayer *L, const float *x, int64_t batch,
                          float *y, int threads, int absmode);
void oracle_backward_dense(const OracleLayer *L, const float *x, const float *dy,
                           int64_t batch, float *dx, float *acc_in,
                           float *acc_grad, int threads, int absmode);
void oracle_forward_sparse(const OracleLayer *L, const int32_t *ptrs,
                           const int32_t *idx, const float *vals, int64_t batch,
                           float *y, int threads, int absmode);
void oracle_backward_sparse(const OracleLayer *L, const float *x,
                            const int32_t *dptrs, const int32_t *didx,
                            const float *dvals, int64_t batch, float *dx,
                            float *acc_in, float *acc_grad, int threads,
                            int absmode);
/* nnz-sampled grad-W, one value per stored synapse in storage order:
 * gw_scattered[elem], gw_tiles[tile*16 + slot].  fp64 accumulation. */
void oracle_sampled_gradw(const OracleLayer *L, const float *x, const float *dy,
                          int64_t batch, float *gw_scattered, float *gw_tiles,
                          int threads, int absmode);

/* ---- backward with the optimizer update (learning_rate != 0) ----
 * disldo_backward (linear_disldo.hpp:466-2113) with deterministic rounding as
 * the deterministic layer classes run it (sili/cpu_backend.cpp:1007-1013),
 * BoundedRMSpropSynapsePolicy and the constants of
 * sili/cpu_backend.cpp:496-528, on a layer without block4 tiles, one thread
 * (the accumulation order of num_cpus = 1).  variant:
 *   0  RMSpropScalePolicy, scales written in the loop (SparseLinearLayer*)
 *   1  RMSpropScalePolicy, DeferredScaleWrite (SparseLinearLayerResync*)
 *   2  NoScalePolicy (SparseLinearLayerNoScale*)
 * The value bytes and the scale state are updated in place; dx, acc_in and
 * acc_grad ACCUMULATE. */
typedef struct {
    float lr;
    int32_t lr_per_row_nnz;
    int32_t damp_by_importance;
    float beta2, eps, beta1, min_decay_frac, max_abs_delta, max_ci, zero_escape_eps;
    int32_t variant;
    /* draws of the stochastic rounding in the sparse-gradient update of block4
     * tiles (the reference rounds those stochastically in every layer class):
     *   0  the reference's per-thread xorshift64* (fp4quant.hpp:174-200) as
     *      fp4_seed_stochastic_rng(draw_seed) leaves it, one step per draw in
     *      call order (draws only for finite |v| < 6)
     *   1  the GPU library's counter draws: splitmix64(draw_seed + id), id =
     *      2 * ((b * n_tiles + t) * 16 + slot) (+1 for the importance) */
    int32_t draw_mode;
    uint64_t draw_seed;
} OracleTrainParams;

/* The block rows' write-back of an optimizer update
 * (Block4Store::merge_row_workspace, block4.hpp:1367-1462): a block row whose
 * stored tiles (sparse-packed or 16 bytes, by tile_sparse) outgrow its
 * reserved tile bytes loses its live slots of lowest |true importance|
 * (decoded importance x importance_scale[row] x output_importance_scale[col]
 * in fp64; the first in (tile, tile row, tile column) order on ties), each
 * eviction re-encoding its tile by its live count, until the row fits; a row
 * that still does not fit counts an overflow event and the bytes beyond its
 * last whole tile that fits. */
typedef struct {
    const uint64_t *tile_alloc; /* [ceil(n_in/4)] reserved tile bytes per block row */
    uint8_t *tile_sparse;       /* [n_tiles] tile_is_sparse, updated */
    uint32_t switch_point;      /* a commit stores a tile sparse-packed iff live <= switch_point */
    uint64_t evicted;           /* out (added to): slots evicted */
    uint64_t overflow_events;   /* out (added to): row_merge_overflow_events */
    uint64_t overflow_bytes;    /* out (added to): row_merge_overflow_bytes_dropped */
} OracleB4Merge;

typedef struct {
    float *value_scale;                   /* [n_in*rank]  */
    float *vs_importance;                 /* [n_in*rank]  */
    float *vs_momentum;                   /* [n_in*rank]  */
    uint32_t *vs_step;                    /* [n_in*rank]  */
    float *output_scale;                  /* [n_out*rank] */
    float *os_importance;                 /* [n_out*rank] */
    uint32_t *os_step;                    /* [n_out*rank] */
    const float *importance_scale;        /* [n_in]  or NULL (ones) */
    const float *output_importance_scale; /* [n_out] or NULL (ones) */
    const int32_t *out_degree;            /* [n_out] */
    int32_t output_scale_trainable;
    float *quant_out;                     /* [nnz] or NULL: each synapse's updated weight code value
                                             before re-quantization */
    float *imp_out;                       /* [nnz] or NULL: its importance (stored units) before it */
    OracleB4Merge *b4;                    /* NULL: block rows taken to have room (no eviction); else
                                             the updates re-encode the tiles they rewrite by live count
                                             and write each block row back as merge_row_workspace */
} OracleTrainState;

/* L supplies structure (its val / scale pointers are not read); val: the
 * layer's value bytes, tiles: its block4 tile bytes (canonical storage order),
 * both updated.  Returns -1 on a layer with tiles when tiles is NULL. */
int oracle_backward_train(const OracleLayer *L, uint8_t *val, uint8_t *tiles, OracleTrainState *S,
                          const float *x, const float *dy, int64_t batch, float *dx,
                          float *acc_in, float *acc_grad, const OracleTrainParams *P);

/* backward_sparse with the optimizer update (sisldo_ops.hpp:589-848, the
 * scattered store; sili/cpu_backend.cpp:587-603): batch rows outer, each
 * synapse with a dy entry in that batch row re-quantized after every step
 * (deterministic rounding, ValueAccessor::set), value_scale stepped once per
 * row after all batch rows.  Output scales, the step variant of the layer
 * class and the importance running stats are not involved.  One thread.
 * dy: CSR with strictly increasing indices per batch row.  S: value_scale,
 * vs_importance, vs_step, output_scale, importance scales read/updated (the
 * rest unused).  Block4 tiles (sisldo_ops.hpp:848-1100; tiles: the layer's
 * tile bytes in canonical order, updated): per batch row, every slot whose dy
 * is nonzero steps its decoded weight and importance (no bounds) and is
 * re-quantized stochastically (draw_mode); the block rows' value_scale step
 * follows, by the row index, step counter (row, 0), no finiteness guards.
 * Returns -1 on a layer with tiles when tiles is NULL. */
int oracle_backward_sparse_train(const OracleLayer *L, uint8_t *val, uint8_t *tiles, OracleTrainState *S, const float *x,
                                 const int32_t *dptrs, const int32_t *didx, const float *dvals, int64_t batch,
                                 float *dx, float *acc_in, float *acc_grad, const OracleTrainParams *P);

/* ---- the reference's synaptogenesis policy ----
 * oracle_build_probes: delta_csr_build_probes (delta_csr_memory.hpp:1309-1426);
 * returns the probe count (entries beyond cap are counted, not written), -1
 * when k <= 0 or the layer is empty.
 * oracle_synap_row_step: delta_csr_synap_row_step (delta_csr_memory.hpp:
 * 1021-1264) on one row, sequential edit semantics; out_degree updated in
 * place; the new structure in the out_* arrays; returns 1/0 as the reference
 * returns true/false.  res_b/res_e (NULL: unlimited): the rows' reserved
 * index bytes and elements; -2 when an insert does not fit (the reference
 * throws; removals and earlier inserts stay applied; fail[0..4] = probe
 * index, column, used bytes, reserved bytes, insertions skipped), -3 when a
 * demotion does not fit (layer as before; fail[0..2] = row, br, bc). */
int64_t oracle_build_probes(const OracleLayer *L, const float *acc_in, const float *acc_grad, int64_t k,
                            int per_row, int32_t *prow, int32_t *pcol, float *pval, int64_t cap);
/* The block4 store's reservations and tile encoding for
 * oracle_synap_row_step2 (block4.hpp:497-946,1170-1290): per block row the
 * reserved index bytes ia, tile slots ea and tile bytes ta (updated), the
 * budgets, switch_point, and tile_is_sparse of the input tiles (canonical
 * order) / of the output tiles. */
typedef struct {
    uint64_t *ia, *ea, *ta;
    uint64_t idx_budget, tile_budget;
    uint32_t switch_point;
    const uint8_t *flags_in;
    uint8_t *flags_out;
    uint64_t dropped; /* out (added to): dropped_growth_events */
} OracleB4Res;
int oracle_synap_row_step(const OracleLayer *L, int64_t row, const int32_t *prow, const int32_t *pcol,
                          const float *pval, int64_t pnnz, int has_probes, float importance_cutoff,
                          int64_t max_row_weights, int64_t max_prune_per_step, float importance_eps,
                          int32_t *out_degree, int32_t *out_ptrs, int32_t *out_cols, uint8_t *out_bytes,
                          int32_t *out_br, int32_t *out_bc, uint8_t *out_tiles, int64_t *n_tiles_out,
                          const uint64_t *res_b, const uint64_t *res_e, int64_t *fail);
/* The same with the block4 store's reservations (b4, see OracleB4Res): a new
 * tile grows its block row without room (get_or_create), a tile's growth
 * beyond the tile budget is dropped (the tile keeps its bytes), and -4 when
 * a new tile's row growth exceeds a budget (the reference throws bad_alloc
 * there: the edits before it and that insert's scattered synapse stay,
 * fail[0] = the probe index). */
int oracle_synap_row_step2(const OracleLayer *L, int64_t row, const int32_t *prow, const int32_t *pcol,
                           const float *pval, int64_t pnnz, int has_probes, float importance_cutoff,
                           int64_t max_row_weights, int64_t max_prune_per_step, float importance_eps,
                           int32_t *out_degree, int32_t *out_ptrs, int32_t *out_cols, uint8_t *out_bytes,
                           int32_t *out_br, int32_t *out_bc, uint8_t *out_tiles, int64_t *n_tiles_out,
                           const uint64_t *res_b, const uint64_t *res_e, int64_t *fail, OracleB4Res *b4);

/* ---- bulk synaptogenesis step (magnitude prune + candidate regrow) ----
 * Output capacities: scattered entries <= nnz + n_cand + 16*n_tiles,
 * tiles <= n_tiles + n_cand.  Outputs are absolute: out_ptrs[n_in+1],
 * out_cols/out_bytes (scattered, row-major, sorted), out_tile_br/bc sorted by
 * (br,bc), out_tile_bytes 16 per tile. */
typedef struct {
    int64_t n_prune_target;
    int64_t n_pruned;
    int64_t n_grown;
    int64_t n_demoted_tiles;
    int64_t n_promoted_tiles;
    int64_t n_scattered;
    int64_t n_tiles;
} OracleSynaptoStats;

int oracle_synapto_step(const OracleLayer *L, float prune_frac,
                        const int32_t *cand_r, const int32_t *cand_c,
                        const float *cand_v, const float *cand_score,
                        int64_t n_cand, int default_imp_code,
                        int32_t *out_ptrs, int32_t *out_cols, uint8_t *out_bytes,
                        int32_t *out_tile_br, int32_t *out_tile_bc,
                        uint8_t *out_tile_bytes, OracleSynaptoStats *stats);

#ifdef __cplusplus
}
#endif
#endif /* SILI_ORACLE_H */
