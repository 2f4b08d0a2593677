/*
 * flare_amd.h -- C ABI of the MI355X (gfx950) sparse-embedding hot path.
 *
 * Plain C: device pointers, sizes, enums and a HIP stream handle (passed as
 * void*).  No torch or other framework types cross this boundary.  Every
 * function returns 0 (FLARE_OK) or a flare_status code and leaves a message
 * for flare_last_error().  All work is enqueued asynchronously on the given
 * stream unless the comment says the call synchronizes.
 *
 * Reference interfaces each entry point replaces are cited as path:line in
 * the fluxway-project/flare tree.
 */
#ifndef FLARE_AMD_H
#define FLARE_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FLARE_ABI_VERSION 3

/* Status codes; the Python layer maps them to the reference's exception
 * classes (src/flare/kernels/backends/gpu_cupy.py:351-354,398-401,479-483). */
typedef enum flare_status {
  FLARE_OK = 0,
  FLARE_ERR_DTYPE = 1,     /* unsupported dtype            -> TypeError    */
  FLARE_ERR_SHAPE = 2,     /* inconsistent sizes           -> ValueError   */
  FLARE_ERR_WIDTH = 3,     /* bad pooled target widths     -> ValueError   */
  FLARE_ERR_ARGUMENT = 4,  /* other invalid argument       -> ValueError   */
  FLARE_ERR_WORKSPACE = 5, /* workspace smaller than asked -> ValueError   */
  FLARE_ERR_HIP = 6,       /* HIP runtime failure          -> RuntimeError */
  FLARE_ERR_LIMIT = 7      /* size beyond supported range  -> ValueError   */
} flare_status;

typedef enum flare_dtype {
  FLARE_FLOAT32 = 0,
  FLARE_FLOAT16 = 1,
  FLARE_BFLOAT16 = 2,
  FLARE_INT32 = 3,
  FLARE_INT64 = 4,
  FLARE_UINT32 = 5,
  FLARE_UINT64 = 6
} flare_dtype;

typedef enum flare_pooling {
  FLARE_POOL_SUM = 0,      /* reference pooling (gpu_cupy.py:96-103)          */
  FLARE_POOL_MEAN = 1,     /* divisor max(#valid,1), jax/layers/embedding.py:124-126 */
  FLARE_POOL_WEIGHTED = 2  /* per-sample weights (no reference counterpart)    */
} flare_pooling;

/* Order of the pooled rows of a CSR batch over T tables and B samples
 * (pooled output and pooled gradient alike).  SAMPLE_MAJOR is one group of T
 * features, [B, T, D] as gather_pooled returns it for target widths (T, M)
 * (contracts.py:63-73).  TABLE_MAJOR packs the T single-feature groups that
 * T separate gather_pooled calls would return, [B, 1, D] each, one after the
 * other: [T, B, D], row t*B + b, the bag order of the CSR batch itself. */
typedef enum flare_layout {
  FLARE_LAYOUT_SAMPLE_MAJOR = 0,
  FLARE_LAYOUT_TABLE_MAJOR = 1,
  /* Flag for flare_pooled_dedup / flare_pooled_backward, OR'ed into
   * FLARE_LAYOUT_TABLE_MAJOR: the caller states that every bag holds exactly
   * one id (offsets[k] == k).  Occurrence i is then pooled row i, so the
   * dedup neither stores nor sorts a gradient row per occurrence.  The dedup
   * checks the statement: any bag of another length sets error bit 1 and
   * rejects the batch (no runs, the update does nothing).  Also taken by
   * flare_gather_pooled_csr.  Ignored with SAMPLE_MAJOR. */
  FLARE_LAYOUT_ONE_ID_PER_BAG = 0x100
} flare_layout;

typedef enum flare_optimizer_kind {
  FLARE_OPT_NONE = 0,            /* write the deduplicated gradient sum only */
  FLARE_OPT_SGD = 1,             /* se.Sgd (dynamic_embedding.py:97-101)      */
  FLARE_OPT_ADAM = 2,            /* se.Adam (dynamic_embedding.py:89-96;
                                    audit_sparse_training.py:460-471)         */
  FLARE_OPT_ROWWISE_ADAGRAD = 3  /* one fp32 accumulator per row              */
} flare_optimizer_kind;

/* Mirrors SparseOptimizerConfig (src/flare/training/components/sparse_table/contracts.py:14-25).
 * Hyper-parameters are doubles, as the Python config holds them; the kernels
 * use float32 lr/eps/beta, float32 (1-beta) and float32 bias corrections
 * 1-beta^step evaluated in double.  weight_decay must be 0 (the only value
 * whose semantics the reference pins). */
typedef struct flare_optimizer {
  int32_t kind;
  int32_t reserved;
  double learning_rate;
  double beta1;
  double beta2;
  double eps;
  double weight_decay;
} flare_optimizer;

/* Thread-local message of the last failing call on this thread. */
const char *flare_last_error(void);
int32_t flare_abi_version(void);

/* ---------------------------------------------------------------------------
 * Gathers (forward).
 * ------------------------------------------------------------------------- */

/* SparseEmbeddingOperator.gather (src/flare/kernels/contracts.py:52-61;
 * CuPy src/flare/kernels/backends/gpu_cupy.py:332-371, kernels :52-73,:108-132).
 * out[slot,:] = emb[inverse[slot],:], or 0 where inverse[slot] == pad_index.
 * emb: [emb_rows, dim] of value_dtype (float32/float16/bfloat16); out likewise
 * [slots, dim].  Slots outside [0, emb_rows) other than pad are written as 0. */
int flare_gather(const void *emb, int32_t value_dtype, int64_t emb_rows,
                 int32_t dim, const int32_t *inverse, int64_t slots,
                 int32_t pad_index, void *out, void *stream);

/* SparseEmbeddingOperator.gather_pooled (contracts.py:63-73; gpu_cupy.py:373-420,
 * kernels :74-107 fp32 and :133-167 fp16).  inverse: padded [batch, features,
 * max_elements] int32 with pad_index marking empty slots.  fp32 accumulation in
 * slot order, output [batch, features, dim] rounded to value_dtype (RNE).
 * pooling: FLARE_POOL_SUM (reference), _MEAN or _WEIGHTED (weights: float32
 * [batch, features, max_elements], required only for _WEIGHTED). */
int flare_gather_pooled(const void *emb, int32_t value_dtype, int64_t emb_rows,
                        int32_t dim, const int32_t *inverse, int64_t batch,
                        int32_t features, int32_t max_elements,
                        int32_t pad_index, int32_t pooling,
                        const float *weights, void *out, void *stream);

/* CSR pooled gather over num_tables tables packed in one [table_rows, dim]
 * array: the ragged layout that materialize_padded_inverse
 * (recipes/recsys/ranking/schema/input.py:23-123) turns into the padded form,
 * consumed here directly.  Bags are table-major, bag k = t*batch + b, with
 * occurrences ids[offsets[k] .. offsets[k+1]) (ids int32 or int64, table-local
 * rows; global row = row_base[t] + id).  row_base: int64 [num_tables + 1],
 * row_base[num_tables] == table_rows; ids outside [0, row_base[t+1] -
 * row_base[t]) contribute nothing.  n = number of ids; offsets are clamped
 * to [0, n] (offsets must start at 0, end at n and not decrease; a violation
 * sets the device error word).  out: [batch, num_tables, dim] for
 * FLARE_LAYOUT_SAMPLE_MAJOR, [num_tables, batch, dim] for _TABLE_MAJOR.
 * _TABLE_MAJOR | FLARE_LAYOUT_ONE_ID_PER_BAG (n == batch * num_tables) reads
 * each bag's id without waiting for its offsets; a bag whose offsets are not
 * (k, k + 1) sets error bit 1 and its row is zeros. */
int flare_gather_pooled_csr(const void *table, int32_t value_dtype,
                            int64_t table_rows, int32_t dim, const void *ids,
                            int32_t id_dtype, int64_t n, const int64_t *offsets,
                            int32_t num_tables, int64_t batch,
                            const int64_t *row_base, int32_t pooling,
                            int32_t layout, const float *weights, void *out,
                            void *stream);

/* ---------------------------------------------------------------------------
 * Deduplication and gradient reduction (backward).  These need a device
 * workspace whose size the matching *_workspace_bytes call returns.
 * Reductions are deterministic: occurrences are stably sorted by key and
 * summed in occurrence order (no floating-point atomics).
 * ------------------------------------------------------------------------- */

size_t flare_scatter_workspace_bytes(int64_t slots, int64_t emb_rows, int32_t dim);

/* SparseEmbeddingOperator.scatter (contracts.py:75-84; gpu_cupy.py:422-458,
 * kernel :168-191).  out[r,:] = sum_{slot: inverse[slot]=r} grad[slot,:];
 * out: float32 [emb_rows, dim] (fully written, untouched rows are 0). */
int flare_scatter(int64_t emb_rows, int32_t dim, const int32_t *inverse,
                  int64_t slots, int32_t pad_index, const float *grad,
                  float *out, void *workspace, size_t workspace_bytes,
                  void *stream);

/* SparseEmbeddingOperator.scatter_pooled (contracts.py:86-96;
 * gpu_cupy.py:460-524, kernels :192-252).  grad: float32 [batch, features,
 * dim]; inverse: [batch, features, max_elements]; slot s takes grad row
 * s / max_elements.  FLARE_ERR_SHAPE when slots != batch*features*max_elements
 * (gpu_cupy.py:479-483). */
int flare_scatter_pooled(int64_t emb_rows, int32_t dim, const int32_t *inverse,
                         int64_t slots, int32_t pad_index, const float *grad,
                         int64_t batch, int32_t features, int32_t max_elements,
                         float *out, void *workspace, size_t workspace_bytes,
                         void *stream);

/* flare_scatter / flare_scatter_pooled with the keyed sums written in the
 * gradient transport dtype: out_dtype FLARE_FLOAT32, or FLARE_BFLOAT16 (the
 * fp32 sums rounded to nearest even as each row is stored).  This fuses the
 * cast the caller runs after scatter_pooled, grad.astype(transport)
 * (recipes/recsys/ranking/workers/train_worker.py:518-522; the CuPy backend's
 * astype, gpu_cupy.py:434,474): out is [emb_rows, dim] of out_dtype. */
int flare_scatter_ex(int64_t emb_rows, int32_t dim, const int32_t *inverse,
                     int64_t slots, int32_t pad_index, const float *grad,
                     void *out, int32_t out_dtype, void *workspace,
                     size_t workspace_bytes, void *stream);
int flare_scatter_pooled_ex(int64_t emb_rows, int32_t dim, const int32_t *inverse,
                            int64_t slots, int32_t pad_index, const float *grad,
                            int64_t batch, int32_t features, int32_t max_elements,
                            void *out, int32_t out_dtype, void *workspace,
                            size_t workspace_bytes, void *stream);

size_t flare_unique_workspace_bytes(int64_t n, int32_t key_dtype);

/* unique_first_occurrence (src/flare/ops/sparse_unique.py:52-77) and the GPU
 * dedup branch (src/flare/runtime/fluxway/workers/sparse_input.py:140-164):
 * unique keys in first-occurrence order, inverse (int32) and first_indices
 * (int64).  values: [n] of key_dtype (int32/uint32/int64/uint64).
 * unique_out must hold n keys; *unique_count (device int64) receives U.
 * key_bound > 0 promises 0 <= key < key_bound (no synchronization; a key
 * outside it sets device error bit 1 and the results are not defined); with
 * key_bound == 0 the call reads the key range back to the host (synchronizes
 * the stream once). */
int flare_unique_first_occurrence(const void *values, int32_t key_dtype,
                                  int64_t n, int64_t key_bound, void *unique_out,
                                  int32_t *inverse_out,
                                  int64_t *first_indices_out,
                                  int64_t *unique_count, void *workspace,
                                  size_t workspace_bytes, void *stream);

/* flare_unique_first_occurrence without a workspace argument and without
 * allocating: no counterpart in the reference; for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid allocation).  The workspace is a fixed scratch array
 * of 48 MiB that every GPU the library runs on holds until the process ends:
 * n up to 1048576 keys of any key dtype (a larger n whose workspace would not
 * fit returns FLARE_ERR_LIMIT).  key_bound > 0 is required (nothing is read
 * back to the host, nothing synchronizes).  Every call on one GPU shares that
 * GPU's array, which keeps the last call's contents (each call clears what
 * must start at zero), so calls that overlap on one GPU (two streams, two
 * threads) race: order them on one stream.  Outputs as
 * flare_unique_first_occurrence. */
int flare_unique_first_occurrence_noalloc(const void *values, int32_t key_dtype,
                                          int64_t n, int64_t key_bound,
                                          void *unique_out, int32_t *inverse_out,
                                          int64_t *first_indices_out,
                                          int64_t *unique_count, void *stream);

/* ---------------------------------------------------------------------------
 * Sparse optimizer update on a dense, row-indexed table shard in HBM.
 *
 * table: [rows, dim] value_dtype.  State (float32):
 *   ROWWISE_ADAGRAD: state0 = accumulator [rows];
 *   ADAM:            state0 = m [rows, dim], state1 = v [rows, dim],
 *                    step = int32 per-row counter [rows];
 *   SGD / NONE:      unused (may be NULL).
 * ------------------------------------------------------------------------- */

size_t flare_sparse_update_workspace_bytes(int64_t n, int64_t rows, int32_t dim);

/* EmbeddingStore.accumulate_gradients(keys, grad) followed by
 * optimizer_step(normalization_steps) (dynamic_embedding.py:481-549; store
 * calls :525,:527,:544,:546).  keys: int64 rows [n] (duplicates allowed; the
 * gradients of equal keys are summed in occurrence order), grad: float32
 * [n, dim].  The summed gradient is divided by normalization_steps before the
 * optimizer.  Keys outside [0, rows) are ignored. */
int flare_sparse_update(void *table, int32_t value_dtype, int64_t rows,
                        int32_t dim, float *state0, float *state1,
                        int32_t *step, const flare_optimizer *optimizer,
                        const int64_t *keys, int64_t n, const float *grad,
                        int32_t normalization_steps, void *workspace,
                        size_t workspace_bytes, void *stream);

/* flare_sparse_update with the gradient in its transport dtype, cast on load
 * instead of in a separate pass (train_worker.py:520-527 and
 * sparse_precision.py:150-192: prepare_sparse_native_gradient casts bf16 / fp32
 * transport to the fp32 native gradient).  grad_dtype: FLARE_FLOAT32 or
 * FLARE_BFLOAT16 (SPARSE_GRADIENT_TRANSPORT_DTYPES, sparse_precision.py:12-14);
 * a bf16 value widens exactly, so the result equals casting first.
 * check_finite != 0 (validate_values=True, sparse_precision.py:121-148):
 * the gradient is checked first; if any element is inf / NaN nothing is
 * updated, *nonfinite_out (device int32, required then) becomes 1 and device
 * error bit 8 is set; otherwise *nonfinite_out becomes 0. */
int flare_sparse_update_ex(void *table, int32_t value_dtype, int64_t rows,
                           int32_t dim, float *state0, float *state1,
                           int32_t *step, const flare_optimizer *optimizer,
                           const int64_t *keys, int64_t n, const void *grad,
                           int32_t grad_dtype, int32_t check_finite,
                           int32_t *nonfinite_out, int32_t normalization_steps,
                           void *workspace, size_t workspace_bytes, void *stream);

/* Timing markers for the calling thread, with no counterpart in the reference
 * (a profiling hook, as NVTX ranges are for CUDA code): while count (0..4) is
 * non-zero, every update entry point called from this thread records
 * events[0] on its stream before the segment sums kernel, events[1] after
 * it, events[2] after the hot-key folds and events[3] after the apply
 * kernel; a null entry records nothing at its point (each record is a
 * marker packet of a few microseconds).  The events are the caller's
 * (hipEvent_t, created and kept alive by the caller until the work is done);
 * count 0 turns the markers off. */
int flare_set_update_events(void *const *events, int32_t count);

/* require_finite_sparse_values (sparse_precision.py:121-148) on the device:
 * *nonfinite_out (device int32) = 1 when any of the count float32 / float16 /
 * bfloat16 elements is inf or NaN, else 0.  Sets device error bit 8 too. */
int flare_check_finite(const void *values, int32_t dtype, int64_t count,
                       int32_t *nonfinite_out, void *stream);

size_t flare_pooled_backward_workspace_bytes(int64_t n, int64_t rows,
                                             int32_t dim);

/* Fused backward of flare_gather_pooled_csr: dedup of the occurrence stream
 * (global row keys row_base[t] + ids[i], i < n == offsets[batch*num_tables]),
 * per-occurrence gradient
 * (pooled_grad[b,t,:], times weights[i] for WEIGHTED or / bag length for
 * MEAN), deterministic segment reduction, then the optimizer update of the
 * table rows -- scatter_pooled (gpu_cupy.py:460-524) + accumulate_gradients +
 * optimizer_step fused.  pooled_grad: float32 [batch, num_tables, dim]
 * (SAMPLE_MAJOR) or [num_tables, batch, dim] (TABLE_MAJOR), as `layout` says.
 * With optimizer->kind == FLARE_OPT_NONE the reduced gradient is written to
 * grad_out [U, dim] in first-occurrence order and the table is not touched.
 * Optional outputs (NULL to skip): unique_out (int64 global rows, first
 * occurrence order), inverse_out (int32 [n]), first_indices_out (int64),
 * unique_count (device int64). */
int flare_pooled_backward(void *table, int32_t value_dtype, int64_t rows,
                          int32_t dim, float *state0, float *state1,
                          int32_t *step, const flare_optimizer *optimizer,
                          const void *ids, int32_t id_dtype, int64_t n,
                          const int64_t *offsets, int32_t num_tables,
                          int64_t batch, const int64_t *row_base,
                          int32_t pooling, int32_t layout, const float *weights,
                          const float *pooled_grad, int32_t normalization_steps,
                          float *grad_out, int64_t *unique_out,
                          int32_t *inverse_out, int64_t *first_indices_out,
                          int64_t *unique_count, void *workspace,
                          size_t workspace_bytes, void *stream);

/* The two halves of flare_pooled_backward, sharing one workspace:
 * flare_pooled_dedup needs only the ids (it can run as soon as the batch is
 * known, e.g. right after the forward), flare_pooled_apply consumes the
 * pooled gradient and the dedup left in the workspace (same n, num_tables,
 * batch, rows, dim and pooling; the layout is the dedup's).  unique_out / first_indices_out /
 * unique_count are written by the dedup, inverse_out by the apply. */
int flare_pooled_dedup(const void *ids, int32_t id_dtype, int64_t n,
                       const int64_t *offsets, int32_t num_tables, int64_t batch,
                       const int64_t *row_base, int64_t rows, int32_t dim,
                       int32_t pooling, int32_t layout, int64_t *unique_out,
                       int64_t *first_indices_out, int64_t *unique_count,
                       void *workspace, size_t workspace_bytes, void *stream);

int flare_pooled_apply(void *table, int32_t value_dtype, int64_t rows, int32_t dim,
                       float *state0, float *state1, int32_t *step,
                       const flare_optimizer *optimizer, int64_t n,
                       int32_t num_tables, int64_t batch, int32_t pooling,
                       const float *weights, const float *pooled_grad,
                       int32_t normalization_steps, float *grad_out,
                       int32_t *inverse_out, void *workspace, size_t workspace_bytes,
                       void *stream);

/* flare_pooled_apply with the pooled gradient in its transport dtype
 * (FLARE_FLOAT32 or FLARE_BFLOAT16, cast on load) and an optional finite
 * check, as flare_sparse_update_ex. */
int flare_pooled_apply_ex(void *table, int32_t value_dtype, int64_t rows, int32_t dim,
                          float *state0, float *state1, int32_t *step,
                          const flare_optimizer *optimizer, int64_t n,
                          int32_t num_tables, int64_t batch, int32_t pooling,
                          const float *weights, const void *pooled_grad,
                          int32_t grad_dtype, int32_t check_finite,
                          int32_t *nonfinite_out, int32_t normalization_steps,
                          float *grad_out, int32_t *inverse_out, void *workspace,
                          size_t workspace_bytes, void *stream);

/* ---------------------------------------------------------------------------
 * Dynamic key -> row map (the dynamic store's lookup_or_insert).
 *
 * Replaces the key index of sparse_embedding.EmbeddingStore as
 * DynamicSparseEmbeddingSPMD drives it: lookup_or_insert(keys, dim)
 * (src/flare/runtime/fluxway/workers/dynamic_embedding.py:397-399), new rows
 * drawn from Uniform(min_val, max_val) (:262-263), reserve(capacity, dim)
 * (:296-302).  Keys are arbitrary int64 except INT64_MIN; rows index a
 * caller-owned table of row_capacity rows.  Each call gives new keys rows
 * row_count, row_count+1, ... in the order of their first occurrence in
 * `keys` and writes their initial values: element (key, c) is
 * lo + (hi - lo) * u with u = 24 bits of splitmix64 mixing of
 * (seed, key, c), scaled to [0, 1), rounded to the storage dtype.
 * Calls on one map must be ordered (one stream).
 * ------------------------------------------------------------------------- */

/* Bytes of a map with `capacity` slots (a power of two in [64, 2^30]); 0 when
 * the capacity is invalid.  Keep the load (keys / capacity) at or below 1/2. */
size_t flare_keymap_bytes(int64_t capacity);

/* Empties a map buffer (no keys, row count 0). */
int flare_keymap_init(void *map, int64_t capacity, void *stream);

/* Device workspace of one lookup_or_insert call over n keys. */
size_t flare_keymap_workspace_bytes(int64_t n);

/* rows_out[i] (int32, optional) = row of keys[i]; values_out[i, :] (optional,
 * storage dtype, [n, dim]) = its values.  insert != 0: missing keys get rows
 * (see above; table required).  insert == 0: missing keys give row -1 and
 * zero values.  A full map or table sets device error bit 4 and leaves the
 * key without a row (-1).  table may be NULL for a row-only lookup. */
int flare_keymap_lookup_or_insert(void *map, int64_t capacity, const int64_t *keys,
                                  int64_t n, int32_t insert, void *table,
                                  int32_t value_dtype, int64_t row_capacity,
                                  int32_t dim, float init_lo, float init_hi,
                                  uint64_t seed, int32_t *rows_out,
                                  void *values_out, void *workspace,
                                  size_t workspace_bytes, void *stream);

/* Re-inserts every key of src (and the row count) into dst, which it first
 * empties: growing a map on reserve(). */
int flare_keymap_rehash(const void *src, int64_t src_capacity, void *dst,
                        int64_t dst_capacity, void *stream);

/* The keys that hold rows and their rows, in slot order: keys_out (int64) and
 * rows_out (int32) need room for every stored key; *count_out (device int64)
 * gets their number.  The store's export_page_images
 * (tests/runtime/test_sparse_storage_limits.py:62-79,
 * tools/validation/audit_sparse_checkpoint.py:33-70) reads keys, values,
 * optimizer states and steps through it. */
size_t flare_keymap_export_workspace_bytes(int64_t capacity);
int flare_keymap_export(const void *map, int64_t capacity, int64_t *keys_out,
                        int32_t *rows_out, int64_t *count_out, void *workspace,
                        size_t workspace_bytes, void *stream);

/* dst[dst_index[i]] = src[src_index[i]] for i < n, rows of row_bytes bytes
 * copied as they are (either index may be NULL: the identity).  Rows outside
 * [0, src_rows) / [0, dst_rows) are skipped and set device error bit 1.  The
 * stores' assign(keys, values) (test_sparse_checkpoint_audit.py:35-39) and
 * page-image export / import move values, optimizer state and step counters
 * with it. */
int flare_copy_rows(const void *src, int64_t src_rows, void *dst, int64_t dst_rows,
                    int64_t row_bytes, const int32_t *src_index,
                    const int32_t *dst_index, int64_t n, void *stream);

/* dst[0 .. bytes) = 0 on the stream, by a fill kernel (not hipMemsetAsync, so
 * that a caller may capture it in a HIP graph).  Replaces the CuPy backend's
 * cudaMemsetAsync (src/flare/kernels/backends/gpu_cupy.py:255-300), which
 * zeroes the outputs of its atomic scatters (:422-524). */
int flare_zero_bytes(void *dst, int64_t bytes, void *stream);

/* dst[i] = src[i] converted between float32, float16 and bfloat16 (widening
 * exact, narrowing round-to-nearest-even) for count elements.  The transport
 * casts of the reference's callers run on it: the keyed gradient sum cast to
 * the bf16 wire dtype (recipes/recsys/ranking/workers/train_worker.py:518-522)
 * and the bf16 -> fp32 native cast (src/flare/runtime/sparse_precision.py:
 * 150-192), as the CuPy backend's astype does (gpu_cupy.py:434,474). */
int flare_convert(const void *src, int32_t src_dtype, void *dst, int32_t dst_dtype,
                  int64_t count, void *stream);

/* A non-blocking stream at default priority, as the CuPy backend keeps one
 * per operator (src/flare/kernels/backends/gpu_cupy.py:253), for hosts with
 * no HIP runtime binding of their own; synchronize and destroy it with the
 * two calls after.  Every entry point takes such a stream (or NULL: the
 * default stream) as its last argument. */
int flare_stream_create(void **stream_out);
int flare_stream_synchronize(void *stream);
int flare_stream_destroy(void *stream);

/* Dense global positions (int32) of the unique ids' first occurrences in a
 * ragged batch: _unique_global_flat_positions
 * (src/flare/runtime/fluxway/workers/sparse_input.py:85-113) on the device.
 * splits[k] (device int64, split_lengths[k] values) for k < levels <= 4:
 * splits[0] maps local rows to level-1 entries, the last level maps entries
 * to flat values.  Flat index first_indices[u] with path (r0, j1..jL) goes to
 * origin_indices[r0] * S_0 + sum_k j_k * S_k, S the suffix products of widths
 * (the dense shape after the row axis, host int64[levels]).  A path outside
 * the splits, a j_k >= widths[k-1] or r0 >= origin_rows gives -1 and sets
 * device error bit 1. */
int flare_nested_global_positions(const int64_t *first_indices, int64_t count,
                                  int32_t levels, const int64_t *const *splits,
                                  const int64_t *split_lengths,
                                  const int64_t *origin_indices, int64_t origin_rows,
                                  const int64_t *widths, int32_t *out, void *stream);

/* Reads back and clears the device-side error word that kernels set: bit 1 an
 * out-of-range index (written as 0 / ignored) or invalid CSR offsets, bit 2 an
 * exhausted spin-wait guard, bit 4 a full key map or table, bit 8 a checked
 * gradient with inf / NaN.  Synchronizes the stream.  Returns the flag bits. */
int32_t flare_take_device_errors(void *stream);

#ifdef __cplusplus
}
#endif

#endif /* FLARE_AMD_H */
