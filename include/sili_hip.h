/*
 * sili_hip.h -- C ABI of the MI355X (gfx950) FP4 delta-CSR sparse linear layer.
 *
 * Drop-in boundary for sili's SparseLinearLayer hot path
 * (SimLeek/sili__new sili/cpu_backend.cpp:349-984, bindings :1506-1743).
 * Plain C: opaque handle, int status codes, thread-local last-error string,
 * plain pointers and sizes, streams passed as void* (a hipStream_t, or NULL
 * for the layer's own stream).  No torch or HIP types appear here.
 *
 * Memory: arguments documented "device" are device pointers; "host" are host
 * pointers.  Compute entry points are asynchronous on the given stream unless
 * documented otherwise; sili_synchronize() waits for the layer's stream.
 * Calls on one layer share its workspaces (staged activations, split-row
 * partial sums and arrival counters): calls on one layer that overlap on
 * different streams race; order them on one stream or with events.
 *
 * Layout conventions (the reference's):
 *   - matrix rows are INPUT neurons: y[b,c] = sum_r x[b,r] * W(r,c)
 *     (linear_disldo.hpp:63-65);
 *   - activations are fp32 [batch, n] row-major (linear_disldo.hpp:41-44);
 *   - scattered value byte = (w_code<<4)|imp_code (fp4quant.hpp:280-383);
 *   - block4 slot byte = (imp_code<<4)|w_code, slot = lj*4+li (block4.hpp:300-312);
 *   - sparse activations are CSR: int32 ptrs[batch+1], int32 indices sorted
 *     ascending within each batch row, fp32 values (sisldo_ops.hpp:372-378).
 */
#ifndef SILI_HIP_H
#define SILI_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes.  The Python binding maps them to the exception types the
 * reference raises (sili/cpu_backend.cpp: std::invalid_argument -> ValueError,
 * std::bad_alloc -> MemoryError, std::runtime_error -> RuntimeError,
 * std::out_of_range -> IndexError). */
enum {
    SILI_OK = 0,
    SILI_ERR_INVALID = 1,   /* ValueError   */
    SILI_ERR_NOMEM = 2,     /* MemoryError  */
    SILI_ERR_RUNTIME = 3,   /* RuntimeError */
    SILI_ERR_RANGE = 4,     /* IndexError   */
    SILI_ERR_HIP = 5        /* RuntimeError (HIP runtime failure) */
};

typedef struct sili_layer sili_layer;

/* Last error message of the calling thread ("" when none). */
const char *sili_last_error(void);

/* ---- lifetime --------------------------------------------------------- */

/* SparseLinearLayer(n_inputs, n_outputs, max_weights, num_cpus)
 * (sili/cpu_backend.cpp:375-447).  max_weights sets the same byte budgets as
 * the reference (index bytes max_weights*8+4096, values max_weights+64,
 * block4 tiles max(4,max_weights/16)*16); loads beyond them fail with
 * SILI_ERR_NOMEM.  device = HIP device ordinal. */
int sili_create(int64_t n_inputs, int64_t n_outputs, int64_t max_weights, int device,
                sili_layer **out);
void sili_destroy(sili_layer *layer);
/* Wait for all work queued on the layer's stream. */
int sili_synchronize(sili_layer *layer);
/* The layer's own hipStream_t (as void*). */
void *sili_stream(sili_layer *layer);

/* ---- construction / state -------------------------------------------- */

/* load_weights(ptrs, indices, vals) (sili/cpu_backend.cpp:859-901): host
 * absolute CSR over input rows; vals are fp4-quantized (fp4quant.hpp:86-126),
 * importance 0.  imp may be NULL; when given it is quantized into the low
 * nibble (delta_csr_memory.hpp:16-93 takes importance per synapse).  Columns
 * must be strictly increasing within a row and < n_outputs.  Replaces the
 * scattered store; the block4 store is left as is. */
int sili_load_weights(sili_layer *layer, const int32_t *ptrs, const int32_t *indices,
                      const float *vals, const float *imp, int64_t nnz);

/* Same, from raw value bytes (w_code<<4 | imp_code), no quantization. */
int sili_load_weight_bytes(sili_layer *layer, const int32_t *ptrs, const int32_t *indices,
                           const uint8_t *bytes, int64_t nnz);

/* load_dense_codes(weight_codes, importance_codes) (sili/cpu_backend.cpp:910-921,
 * delta_csr_memory.hpp:841-945): host uint8 [n_in*n_out] code matrices; every
 * 4x4 block becomes a block4 tile (byte = w | imp<<4), replacing the block4
 * store. */
int sili_load_dense_codes(sili_layer *layer, const uint8_t *weight_codes,
                          const uint8_t *importance_codes);

/* Block4 store from a tile list (no reference counterpart as one call: the
 * reference builds the same store tile by tile with Block4Store::get_or_create,
 * block4.hpp:1168-1188).  host int32 br[n], bc[n] (any order, no duplicates),
 * host uint8 tile_bytes[16*n] in slot order lj*4+li. Replaces the block4 store. */
int sili_load_block4_tiles(sili_layer *layer, const int32_t *br, const int32_t *bc,
                           const uint8_t *tile_bytes, int64_t n_tiles);

/* Seeded synthetic layer built on the device (no reference counterpart: the
 * benchmark workloads of BASELINE config 4 are too large to build on the
 * host; the reference's own builds go through load_weights).  Synapse (r, c)
 * exists iff a 64-bit hash of (seed, r, c) falls below keep_prob; its weight
 * is drawn from |N(0, sigma)| conditioned on |w| >= sigma * Phi^-1(tail_q)
 * (tail_q = 0.5: plain half-normal) with a random sign, then quantized with
 * the reference's per-row recipe (s_r = fl32(max_row|w| / 6), code =
 * fp4_encode(w / s_r), sili/sparse_rnn.py:1022-1037; importance 0).  Replaces
 * the scattered store and the value scales (rank must be 1); the synapse
 * count goes to *nnz_out (may be NULL).  Synchronous. */
int sili_load_synthetic(sili_layer *layer, uint64_t seed, double keep_prob, float sigma, float tail_q,
                        int64_t *nnz_out);

/* set_scale_rank(k) (sili/cpu_backend.cpp:455-461): 1 <= k <= 4, else
 * SILI_ERR_INVALID.  Resets scales to the reference defaults (component 0 = 1,
 * others 0; delta_csr_types.hpp:1116-1121). */
int sili_set_scale_rank(sili_layer *layer, int rank);
int sili_get_scale_rank(const sili_layer *layer);

/* Bulk set_value_scale_raw_k / set_output_scale_raw_k /
 * set_importance_scale_raw / set_output_importance_scale_raw
 * (sili/cpu_backend.cpp:792-806, delta_csr_types.hpp:1013-1196).
 * host fp32, value/output scales laid out [n*rank] (row-major per
 * component).  Setting output scales marks them trainable, like
 * set_output_scale_raw (delta_csr_types.hpp:1190-1196). */
int sili_set_value_scale(sili_layer *layer, const float *vs);
int sili_set_output_scale(sili_layer *layer, const float *os);
int sili_set_importance_scale(sili_layer *layer, const float *is);
int sili_set_output_importance_scale(sili_layer *layer, const float *ois);
/* host fp32 outputs, same layouts. */
int sili_get_value_scale(const sili_layer *layer, float *vs);
int sili_get_output_scale(const sili_layer *layer, float *os);

/* ---- compute ------------------------------------------------------------ */

/* forward_dense (sili/cpu_backend.cpp:475-492, linear_disldo.hpp:68-345):
 * device x [batch,n_in] -> device y [batch,n_out] (overwritten). */
int sili_forward_dense(sili_layer *layer, const float *x, int64_t batch, float *y,
                       void *stream);

/* forward_dense_noalloc: no counterpart in the reference.  For callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc): the same y as sili_forward_dense
 * (within the fp32 bar), computed without any device allocation.  The
 * feature-major copy of x lives in a per-device scratch of 32 MiB held by the
 * library until the process ends, so n_inputs * batch <= 8388608 for
 * batch > 1 (SILI_ERR_INVALID otherwise).  It reads only structures built at
 * load (the segment gathers), does not keep x as the stored forward input
 * (a following backward_dense must pass x), records no profiler events, and
 * shares the scratch with every other call on the same GPU: calls that overlap
 * on one GPU race.  While synap_row_step / synap_step edits are still pending
 * on the layer (they are written by the next other entry point, and writing
 * them allocates), it returns SILI_ERR_INVALID without computing anything:
 * call sili_synchronize first. */
int sili_forward_dense_noalloc(sili_layer *layer, const float *x, int64_t batch, float *y,
                               void *stream);

/* backward_dense (sili/cpu_backend.cpp:496-529, linear_disldo.hpp:462-2113):
 * dx [batch,n_in] = W^T-gather of dy (overwritten).  x may be NULL: then the
 * input of the last forward_dense on this layer is used, as the reference's
 * backward_dense uses its stored last_input (available for batch > 1; with
 * batch 1 pass x).  Always accumulates neuron_input_accum += sum_b|x| and
 * neuron_grad_accum += sum_b|dy| (linear_disldo.hpp:515-520).  When gw_s /
 * gw_b are non-NULL (learning_rate 0 only), also writes the nnz-sampled
 * grad-W (see sili_sampled_gradw).  learning_rate != 0 runs the optimizer
 * update with the binding's defaults, as sili_backward_dense_train with
 * lr_per_row_nnz 0, damp_by_importance 1, beta2 0.999, eps 1e-8. */
int sili_backward_dense(sili_layer *layer, const float *x, const float *dy, int64_t batch,
                        float *dx, float *gw_s, float *gw_b, float learning_rate,
                        void *stream);

/* backward_dense with the optimizer update (sili/cpu_backend.cpp:496-529;
 * disldo_backward, linear_disldo.hpp:466-2113, with RMSpropScalePolicy, no
 * deferred scale write, BoundedRMSpropSynapsePolicy, beta1 0.9,
 * min_decay_frac 0, max_abs_delta 2, max_ci 100, zero_escape_eps 0.1): for
 * every synapse, batch-sequential RMSprop steps on its stored weight code and
 * importance, re-quantized in place (deterministically or stochastically,
 * sili_set_stochastic_rounding); dx from the updated weights; the value
 * scales' RMSprop step, the Adam step of rows without synapses, and the output
 * scales' step when they are trainable.  batch <= 1024.  Block4 tiles (FP4,
 * linear_disldo.hpp:962-1951): every slot of a tile steps the same way, rows
 * count n_tiles(block row) * 4 synapses, tiles whose 4 columns are in range
 * sum their per-step row terms in the reference's 4-lane order, and the block
 * rows' scale step follows the scattered one; the reference's eviction of
 * live slots when a block row outgrows its reserved bytes has no analogue
 * (the device store is compact and always has room).
 * learning_rate 0 is plain backward_dense. */
int sili_backward_dense_train(sili_layer *layer, const float *x, const float *dy, int64_t batch,
                              float *dx, float learning_rate, int lr_per_row_nnz,
                              int damp_by_importance, float beta2, float eps, void *stream);

/* The scale-update variant of the layer's optimizer update, as the reference's
 * layer classes fix it (sili/cpu_backend.cpp:992-1013):
 *   0 (default) RMSprop steps on the scales inside the loop; the stored code is
 *     stepped by g * S (SparseLinearLayer[Deterministic]);
 *   1 DeferredScaleWrite: true-units weights stepped by g, codes stored under
 *     the scales in effect after the call (SparseLinearLayerResync[Deterministic]);
 *   2 NoScalePolicy: the scales take no step (rows without synapses still do)
 *     (SparseLinearLayerNoScale[Deterministic]). */
int sili_set_update_variant(sili_layer *layer, int variant);

/* Rounding of the update's re-quantization: 1 (default, as the reference's
 * SparseLinearLayer, sili/cpu_backend.cpp:992) stochastic -- unbiased dithered
 * rounding (fp4quant.hpp:210-265) driven by a counter-based generator of this
 * layer (splitmix64 of seed, call and synapse), reproducible for a given seed
 * and call sequence; 0 deterministic round-to-nearest, as
 * SparseLinearLayerDeterministic (sili/cpu_backend.cpp:1007). */
int sili_set_stochastic_rounding(sili_layer *layer, int on);
/* Restart this layer's rounding generator at seed (fp4_seed_stochastic_rng,
 * fp4quant.hpp:186-188, is the reference's per-thread counterpart). */
int sili_seed_stochastic_rounding(sili_layer *layer, uint64_t seed);
/* The scales' optimizer state (delta_csr_types.hpp:1127-1215), host outputs,
 * [n*rank] like the scales; any pointer may be NULL.  Zero before the first
 * update. */
int sili_get_scale_state(const sili_layer *layer, float *vs_importance, float *os_importance,
                         float *vs_momentum, uint32_t *vs_step, uint32_t *os_step);

/* nnz-pattern-sampled grad-W: gw_s[e] = sum_b x[b,r(e)]*dy[b,c(e)] for every
 * scattered synapse e in storage order; gw_b[16*t + slot] likewise for every
 * slot of block4 tile t (tile storage order, slot = lj*4+li).  The reference
 * consumes g = dy*x per synapse inside its optimizer
 * (linear_disldo.hpp:811-882) and never materialises it. */
int sili_sampled_gradw(sili_layer *layer, const float *x, const float *dy, int64_t batch,
                       float *gw_s, float *gw_b, void *stream);

/* forward_sparse (sili/cpu_backend.cpp:571-585, sisldo_ops.hpp:198-551):
 * device CSR input (ptrs[batch+1], indices[nnz_x], values[nnz_x];
 * nnz_x must equal ptrs[batch]) -> device y [batch,n_out] (overwritten). */
int sili_forward_sparse(sili_layer *layer, const int32_t *ptrs, const int32_t *indices,
                        const float *values, int64_t nnz_x, int64_t batch, float *y,
                        void *stream);

/* backward_sparse (sili/cpu_backend.cpp:587-603, sisldo_ops.hpp:589-1104):
 * dense x [batch,n_in], sparse dy CSR (nnz_dy = dy_ptrs[batch], indices
 * strictly increasing per batch row) -> device dx [batch,n_in] (overwritten);
 * accumulates neuron_input_accum / neuron_grad_accum.  learning_rate != 0
 * also runs the optimizer update, as sili_backward_sparse_train with
 * lr_per_row_nnz 0, damp_by_importance 1, beta2 0.999, eps 1e-8. */
int sili_backward_sparse(sili_layer *layer, const float *x, const int32_t *dy_ptrs,
                         const int32_t *dy_indices, const float *dy_values, int64_t nnz_dy,
                         int64_t batch, float *dx, float learning_rate, void *stream);

/* backward_sparse with the optimizer update (disldo_backward_sparse_grad,
 * sisldo_ops.hpp:589-848): batch rows in order; a synapse whose column has a
 * dy entry in a batch row takes an RMSprop step in true units and is
 * re-quantized (round to nearest, whatever the layer's rounding setting)
 * before the next batch row; each row's value scale (slot r, step counter
 * (r, 0)) takes one bias-corrected RMSprop step after all batch rows.  Output
 * scales are not updated.  batch <= 1024.  Block4 tiles (sisldo_ops.hpp:
 * 848-1100), after the scattered section: per batch row every slot whose dy
 * entry is nonzero takes the same unbounded step and is re-quantized
 * stochastically in every layer class, as the reference does (draws
 * splitmix64 of the call seed and (batch row, tile, slot), reproducible
 * under sili_seed_stochastic_rounding); then the block rows' value-scale
 * step.  learning_rate 0 is plain backward_sparse. */
int sili_backward_sparse_train(sili_layer *layer, const float *x, const int32_t *dy_ptrs,
                               const int32_t *dy_indices, const float *dy_values, int64_t nnz_dy,
                               int64_t batch, float *dx, float learning_rate, int lr_per_row_nnz,
                               int damp_by_importance, float beta2, float eps, void *stream);

/* ---- synaptogenesis ----------------------------------------------------- */

/* The reference's own policy (sili/cpu_backend.cpp:606-634).
 * sili_build_probes: delta_csr_build_probes (delta_csr_memory.hpp:1309-1426)
 *   over the layer's neuron_input_accum / neuron_grad_accum: the top-k input
 *   rows by accumulator, crossed with the top-k outputs (shared, or per row
 *   among the columns the row lacks when per_row), pairs already stored in
 *   the scattered store skipped, score = acc_in[r] * acc_grad[c].  k <= 0
 *   zeroes the probe count only, as the reference does.
 * sili_get_probes: the probe list (count to *n, up to cap entries copied).
 * sili_synap_row_step: delta_csr_synap_row_step (delta_csr_memory.hpp:
 *   1021-1264) on row *current_row % n_inputs; *current_row advances (mod
 *   n_inputs) as in the reference.  Removes the row's lowest-importance
 *   synapses (scattered and block4) below importance_cutoff (importance floored
 *   at importance_eps for that test only) or beyond max_row_weights, at most
 *   max_prune_per_step; grows the row's probes by descending score into the
 *   capacity left, weight 0 and importance = score; block4 demotion and
 *   promotion as the reference.  *did: 0 when the row holds nothing and there
 *   are no probes.  Each insert is checked against the row's reservation
 *   (sili_export_layout) as delta_csr_row_insert_col checks it
 *   (delta_csr_memory.hpp:498-585): when one does not fit, the removals and
 *   the inserts before it stay applied, the call returns SILI_ERR_RUNTIME with
 *   the reference's message (:1236-1250) and the cursor does not advance.
 *   When a demotion would not fit (block4_demote_tile, :949-999) the call
 *   returns SILI_ERR_RUNTIME with the layer unchanged (the reference leaves
 *   that tile half demoted).
 * sili_synap_step: the same on the layer's own cursor (synap_step).
 * sili_get_out_degree: out_degree [n_outputs] as the reference keeps it: the
 *   scattered synapses per column after a load, then +1 / -1 per
 *   synap_row_step insert / removal entry (delta_csr_memory.hpp:1216,1246).
 *   It sets the output scales' learning-rate divisor in the update. */
int sili_build_probes(sili_layer *layer, int64_t k, int per_row);
int sili_get_probes(sili_layer *layer, int64_t *n, int32_t *rows, int32_t *cols, float *scores, int64_t cap);
int sili_synap_row_step(sili_layer *layer, int64_t *current_row, float importance_cutoff,
                        int64_t max_row_weights, int64_t max_prune_per_step, float importance_eps,
                        int *did);
int sili_synap_step(sili_layer *layer, float importance_cutoff, int64_t max_row_weights,
                    int64_t max_prune_per_step, float importance_eps, int *did);
int sili_get_out_degree(sili_layer *layer, int32_t *out);

/* Bulk synaptogenesis step, on the GPU.  Selection policy (new; the reference
 * prunes by importance row by row, delta_csr_memory.hpp:1019-1258): prune the
 * round(prune_frac*N) stored synapses (scattered + live block4 slots) with the
 * smallest |dec(code)*S(r,c)|, ties by (row, col) ascending; regrow as many
 * at the host candidates (cand_rows/cols/vals, optional cand_scores), taking
 * the first valid ones in list order (in range, not stored, not just pruned,
 * not a repeat).  A new synapse's code is fp4_encode(val/S(r,c)); its
 * importance code is fp4_encode(score), or default_imp_code without scores.
 * Structural rules follow the reference: a tile whose live count drops below
 * 2 is demoted (delta_csr_memory.hpp:949-999), an insert into a window that
 * holds a tile writes the tile (:620-646), a window that ends up with >= 2
 * scattered synapses after an insert is promoted (:648-700).  The delta-CSR,
 * block4 store and derived device structures are rebuilt by device scan,
 * sort and compaction.  host candidate arrays; results (host) in out_stats[7]:
 * target, pruned, grown, demoted tiles, promoted tiles, scattered nnz, tiles.
 * Synchronous. */
int sili_synapto_step(sili_layer *layer, float prune_frac, const int32_t *cand_rows,
                      const int32_t *cand_cols, const float *cand_vals,
                      const float *cand_scores, int64_t n_cand, int default_imp_code,
                      int64_t *out_stats);

/* ---- the reference's scattered reservations (DeltaCSRLayout) -------------
 * The device store is compact; the layer keeps, per row, the index bytes and
 * value elements the reference's store would reserve, so that inserts run out
 * of room and growth meets the budget (max_weights * 8 + 4096 index bytes,
 * max_weights + 64 values, grown by loads) where the reference's do.
 * Loads reserve as delta_csr_from_absolute with blank_fraction 0.2
 * (delta_csr_memory.hpp:16-93); the bulk sili_synapto_step, which has no
 * reference counterpart, grows a row's reservation to its content when needed.
 * sili_compact: compact() (sisldo_ops.hpp:44-96, sili/cpu_backend.cpp:737-748).
 * sili_expand_headroom[_to]: sisldo_ops.hpp:127-186 (SILI_ERR_NOMEM beyond
 *   the budget, layer unchanged).  compact and expand re-encode every
 *   scattered value byte as the reference's rebuild does (code 8 -> 0).
 * sili_equalize_to_capacity: sili/cpu_backend.cpp:684-729 (target_bytes 0:
 *   5 * target_elems + 4); SILI_ERR_NOMEM when a row's growth exceeds the
 *   budget, the rows before it grown.
 * sili_equalizer_step: equalizer_step (sili/cpu_backend.cpp:646-657): the
 *   scattered store's step (delta_csr_memory.hpp:295-306), then the block4
 *   store's (Block4Store::equalize_step, block4.hpp:1208-1220).
 * sili_export_layout: the reference's byte_start [n_in+1], byte_end [n_in],
 *   elem_start [n_in+1], elem_end [n_in]; any may be NULL. */
int sili_compact(sili_layer *layer);
int sili_expand_headroom(sili_layer *layer, float blank_fraction);
int sili_expand_headroom_to(sili_layer *layer, int64_t min_nnz_per_row, float blank_fraction);
int sili_equalize_to_capacity(sili_layer *layer, int64_t target_elems_per_row, int64_t target_bytes_per_row);
int sili_equalizer_step(sili_layer *layer);
int sili_export_layout(sili_layer *layer, uint64_t *byte_start, uint64_t *byte_end, uint64_t *elem_start,
                       uint64_t *elem_end);

/* No counterpart in the reference: a test hook.  Digests (FNV-1a) of the
 * layer's internal stores -- [0] canonical scattered, [1] its shadow, [2]
 * canonical block4 (with tile_is_sparse), [3] its shadow, [4] the shadow's
 * entry permutation (0 when not kept), [5] the block4 shadow's tile
 * permutation -- each over its sizes, row starts, index bytes, values or
 * tiles, work items and split-row list.  Two layers with equal digests hold
 * the same structure byte for byte (used to compare a row patch with a full
 * rebuild). */
int sili_debug_store_digest(sili_layer *layer, uint64_t digest[6]);

/* ---- accumulators ------------------------------------------------------- */

/* neuron_input_accum / neuron_grad_accum (sili/cpu_backend.cpp:946-951):
 * host copies (n_in / n_out fp32).  Synchronous. */
int sili_get_accumulators(sili_layer *layer, float *acc_in, float *acc_grad);
/* zero_accum() (sili/cpu_backend.cpp:840-843). */
int sili_zero_accum(sili_layer *layer);

/* ---- introspection / export (parity) ------------------------------------ */

typedef struct {
    int64_t n_inputs, n_outputs;
    int64_t nnz_scattered;     /* stored scattered synapses */
    int64_t index_bytes;       /* ULEB128 bytes of the scattered store */
    int64_t n_tiles;           /* block4 tiles */
    int64_t block_index_bytes; /* ULEB128 bytes of the block4 store */
    int64_t live_block4;       /* live (byte != 0) block4 slots */
    int64_t n_segments;        /* decode work items of the scattered store */
    int32_t scale_rank;
    int32_t has_nonfinite;     /* a weight code 8 (NaN) or non-finite scale */
    int32_t stream_canonical;  /* batch-1 stream copy of the canonical store is built */
    int32_t stream_shadow;     /* ... of the shadow (forward) store */
    int32_t split_combined;    /* split rows summed in item order, not with float atomics
                                  (SILI_SPLIT_COMBINE=1 when the store was built): bit 0 the
                                  canonical store, bit 1 the shadow store */
    int32_t pad0;
    int64_t short_rows_canonical; /* short rows (whole rows of <= 28 index bytes) the float4
                                     gather packs up to 16 to a wave, canonical store (0 until
                                     a gather at batch 4..64 has used them, or when fewer than a
                                     quarter of the work items are such rows) */
    int64_t short_rows_shadow;    /* ... of the shadow store */
} sili_info;
int sili_get_info(sili_layer *layer, sili_info *out);

/* Scattered store exactly as held on the device (compact: no headroom):
 * host uint64 row_byte_start[n_in+1], row_elem_start[n_in+1],
 * uint8 idx[index_bytes], uint8 val[nnz_scattered].  NULL skips an array.
 * Synchronous.  (Reference equivalent: DeltaCSRWeights after compact(),
 * sisldo_ops.hpp:44-96.) */
int sili_export_scattered(sili_layer *layer, uint64_t *row_byte_start,
                          uint64_t *row_elem_start, uint8_t *idx, uint8_t *val);

/* Block4 store: host int32 br[n_tiles], bc[n_tiles] in storage order, uint8
 * tiles[16*n_tiles], uint64 brow_byte_start/brow_tile_start [ceil(n_in/4)+1],
 * uint8 bidx[block_index_bytes].  NULL skips an array.  Synchronous. */
int sili_export_block4(sili_layer *layer, int32_t *br, int32_t *bc, uint8_t *tiles,
                       uint64_t *brow_byte_start, uint64_t *brow_tile_start,
                       uint8_t *bidx);

/* Device decode of the scattered store (ULEB128 prefix-scan decode + FP4
 * dequant): host int32 cols[nnz_scattered] and fp32 w_true[nnz_scattered]
 * = fl32(dec(code)*S(r,c)) in storage order.  Either may be NULL. Synchronous. */
int sili_decode_scattered(sili_layer *layer, int32_t *cols, float *w_true);

/* Combined absolute CSR, scattered + live block4 slots, columns ascending per
 * row, decoded stored values (get_ptrs/get_indices/get_weights_vals/
 * get_importance, sili/cpu_backend.cpp:956-983,
 * delta_csr_memory.hpp:127-213).  Call with NULL outputs to get the count in
 * *n_out_entries.  host outputs.  Synchronous. */
int sili_export_absolute(sili_layer *layer, int32_t *ptrs, int32_t *indices, float *w,
                         float *imp, int64_t *n_out_entries);

/* ---- measurement (no reference counterpart: the reference is timed with
 * ad-hoc std::chrono harnesses, scripts/bench_block4_vs_dense_fp4.cpp:58-68) --
 * While enabled, every hot-path kernel the layer launches carries a hipEvent
 * pair that the runtime stamps with that dispatch's own begin and end
 * (hipExtLaunchKernel on the stream it runs on: the kernel's time alone, no
 * queue gaps); sili_profile_read synchronizes, aggregates per
 * "<op>:<kernel>" name in first-seen order, and clears the records.  The
 * backward with grad-W buffers reports its fused pass as "bwd:gather_gradw". */
typedef struct {
    char name[56];
    int64_t count;
    double total_ms, min_ms, max_ms;
} sili_prof_entry;
int sili_profile_enable(sili_layer *layer, int enable);
int sili_profile_read(sili_layer *layer, sili_prof_entry *out, int max_entries, int *n_entries);

/* ---- block4 tile encoding (block4.hpp:332-388, 1016-1031) ---------------
 * The reference stores a tile with <= switch_point (default 10) live slots
 * sparse-packed: [count][ceil(count/2) bytes of 4-bit slot positions, even
 * index in the high nibble][count slot bytes].  The device computes on dense
 * 16-byte tiles and keeps per tile the encoding the reference's store would
 * hold it in (tile_is_sparse): re-encoded by its live count when loaded,
 * promoted, given an insert, or rewritten by an optimizer update; a removal
 * leaves a dense tile dense.  Export, canonical tile order, rows without
 * headroom: tile_is_sparse [n_tiles], tile_data [*nbytes],
 * tile_byte_start [ceil(n_inputs/4)+1]; any output may be NULL. */
int sili_export_block4_packed(sili_layer *layer, uint8_t *tile_is_sparse, uint8_t *tile_data,
                              uint64_t *tile_byte_start, int64_t *nbytes);
/* ---- block4 reservations (block4.hpp:1016-1031, 497-946) -----------------
 * The device store is compact; beside it the layer keeps, per block row, the
 * block-column index bytes, tile slots and tile bytes the reference's
 * Block4Store would reserve, with its budgets (max_weights * 8 + 4096 and
 * max(4, max_weights / 16) * 16 from the constructor; load_dense_codes sets
 * its own, delta_csr_memory.hpp:884-905), under the reference's rules: a new
 * tile (a load's or a promotion's) grows a row without room by
 * block4_ensure_row_headroom, a growth beyond a budget is SILI_ERR_NOMEM, a
 * tile's growth beyond the tile budget is dropped and counted
 * (dropped_growth_events); load_dense_codes reserves 20 % + 16 bytes per row
 * (block4_expand_headroom).  The optimizer updates write each block row back
 * as merge_row_workspace does (block4.hpp:1367-1462): a row whose stored
 * tiles outgrow its reserved tile bytes loses its live slots of lowest
 * |importance code x importance_scale[row] x output_importance_scale[col]|
 * until it fits.  sili_load_block4_tiles (no counterpart) reserves as its
 * tiles placed one by one in canonical order would, and refuses with
 * SILI_ERR_NOMEM what would exceed the budgets.  The bulk sili_synapto_step
 * (no counterpart) grows a row's reservations to its content when needed.
 * sili_expand_block4_headroom: expand_block4_headroom (sili/cpu_backend.cpp:
 *   932-934, delta_csr_memory.hpp:767-823): tile bytes = used + (size_t)(used
 *   * f) + 16 per block row; SILI_ERR_NOMEM beyond the tile budget (layer
 *   unchanged).
 * sili_compact_block4: compact_block4 (:941-943): tile bytes = used.
 * sili_export_block4_layout: per block row [ceil(n_inputs/4)] the reserved
 *   index bytes, tile slots and tile bytes, and the used ones; out[6]:
 *   dropped_growth_events, row_merge_overflow_events,
 *   row_merge_overflow_bytes_dropped, the index and tile budgets, and the
 *   slots the updates' write-back evicted.  Any pointer may be NULL. */
int sili_expand_block4_headroom(sili_layer *layer, float blank_fraction);
int sili_compact_block4(sili_layer *layer);
int sili_export_block4_layout(sili_layer *layer, uint64_t *ia, uint64_t *ea, uint64_t *ta, uint64_t *ui,
                              uint64_t *ue, uint64_t *ut, uint64_t *out);
/* Block4View (sili/cpu_backend.cpp:43-98): the store's counters;
 * alloc_bytes is the sum of the block rows' reserved tile bytes. */
typedef struct {
    int64_t tiles, synapses;
    uint32_t switch_point;
    int64_t used_bytes, alloc_bytes;
    int64_t dropped_growth_events, row_merge_overflow_events, row_merge_overflow_bytes_dropped;
} sili_block4_stats;
int sili_block4_view(sili_layer *layer, sili_block4_stats *out);
/* Block4View.switch_point setter: affects later encodings only, as the
 * reference's; values above 10 are refused (the reference's pack buffer is
 * 16 bytes, block4.hpp:332-340). */
int sili_set_switch_point(sili_layer *layer, uint32_t switch_point);

/* ---- group frame-of-reference index (prototypes/for_delta_encoding/
 * README.md:18-40, for_encoding_bench.cpp:31-96) ----------------------------
 * A derived copy of the canonical store's column indices in the reference
 * prototype's FOR format: per row, groups of group_size (8, 16, 32 or 64)
 * columns, each a tier byte (0/1/2 = 1/2/4 bytes per offset) and group_size
 * little-endian offsets from the group start (the previous group's last
 * column, 0 for a row's first group); a short last group repeats its last
 * offset.  Built on request, dropped when the store is rebuilt (the ULEB128
 * stream stays the source of truth). */
int sili_build_for_index(sili_layer *layer, int group_size);
/* Host copies: row_byte_start [n_inputs+1] (may be NULL), bytes [*nbytes]
 * (may be NULL to query the size). */
int sili_export_for_index(sili_layer *layer, uint64_t *row_byte_start, uint8_t *bytes,
                          int64_t *nbytes);
/* Every canonical column (int32, storage order) into device cols, decoded
 * from the ULEB128 stream (use_for_index 0; DeltaCSRRowCursor,
 * delta_csr_types.hpp:801-832) or from the FOR index: 1, one lane per slot
 * with the wave's group bytes loaded as coalesced dwords; 2, one thread per
 * group (G 8 and 16) or one thread per slot with byte loads (G 32 and 64), kept
 * for comparison.  Other values: SILI_ERR_INVALID.  Profiled as "index:for" /
 * "index:uleb". */
int sili_decode_columns(sili_layer *layer, int32_t *cols, int use_for_index, void *stream);

/* ---- module utilities (device buffers; synchronous on `stream`) -----------
 * fp4_quantize_array (sili/cpu_backend.cpp:3157-3172): codes[i] =
 * fp4_encode(x[i]) (fp4quant.hpp:86-126), n elements. */
int sili_fp4_quantize(const float *x, int64_t n, uint8_t *codes, void *stream);
/* dense_to_csr (sili/cpu_backend.cpp:3075-3116): x [rows, cols] row-major ->
 * CSR of the entries with x > threshold or x < -threshold, in row-major
 * order; ptrs [rows+1].  *nnz receives the entry count; indices/values are
 * written when it is <= capacity (else SILI_ERR_RANGE, ptrs still written). */
int sili_dense_to_csr(const float *x, int64_t rows, int64_t cols, float threshold, int32_t *ptrs,
                      int32_t *indices, float *values, int64_t capacity, int64_t *nnz, void *stream);
/* dense_to_top_k_csr (sili/cpu_backend.cpp:3118-3150, csr.hpp:405-505): the
 * min(k, rows*cols) entries of largest |x| over the whole flattened array
 * (a global budget, as the reference's), as a CSR in row-major order;
 * indices/values hold min(k, rows*cols) entries, ptrs rows+1.  Equal
 * magnitudes at the cut keep the lowest flat index (the reference leaves
 * that order to its per-thread partial sorts); NaN ranks above every
 * finite value. */
int sili_dense_to_top_k_csr(const float *x, int64_t rows, int64_t cols, int64_t k, int32_t *ptrs,
                            int32_t *indices, float *values, int64_t *nnz, void *stream);
/* Layer-free device buffers for the utilities above (hipMemcpyDefault). */
int sili_buffer_alloc(int device, size_t bytes, void **out);
int sili_buffer_free(int device, void *ptr);
int sili_buffer_copy(int device, void *dst, const void *src, size_t bytes);

/* ---- device memory helpers (for callers without HIP headers) ------------ */
int sili_device_alloc(sili_layer *layer, size_t bytes, void **out);
int sili_device_free(sili_layer *layer, void *ptr);
int sili_memcpy_h2d(sili_layer *layer, void *dst, const void *src, size_t bytes);
int sili_memcpy_d2h(sili_layer *layer, void *dst, const void *src, size_t bytes);
int sili_memset_device(sili_layer *layer, void *dst, int value, size_t bytes);
/* Page-locked host memory (hipHostMalloc): copies from and to it run as DMA
 * without a staging copy.  No counterpart in the reference (a CPU library);
 * for binding layers that hand host arrays across the boundary. */
int sili_host_alloc(size_t bytes, void **out);
int sili_host_free(void *ptr);
/* Host -> device copy ordered on the layer's stream (after the work queued on
 * it, before the work queued after it), without waiting for it: the source
 * must stay unchanged until the stream has passed the copy (sili_synchronize,
 * or an ordered device -> host copy, returns).  From page-locked memory
 * (sili_host_alloc) it is one copy kernel on the stream, which reads the host
 * pages directly; from pageable memory, the runtime's staged copy. */
int sili_memcpy_h2d_ordered(sili_layer *layer, void *dst, const void *src, size_t bytes);
/* Device -> host copy ordered on the layer's stream; returns when it has
 * landed (one wait for the stream).  Into page-locked memory it is one copy
 * kernel on the stream, which writes the host pages directly. */
int sili_memcpy_d2h_ordered(sili_layer *layer, void *dst, const void *src, size_t bytes);

#ifdef __cplusplus
}
#endif
#endif /* SILI_HIP_H */
