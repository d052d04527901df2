/*
 * cti_ebag.h — C ABI of the MI355X (gfx950) fused sparse-feature embedding-bag path.
 *
 * The path pools F variable-length sparse fields ("slots") of a batch of B samples into
 * one dense row per sample:  out[b, col_f : col_f + D_f] = pool_{i in bag(b, f)} table_f[clamp(v_i)].
 *
 * Reference interfaces replaced (paths relative to the reference repository):
 *   - online_best/infer.py:793-827   Triton kernel fused_all_slots_embedding_kernel
 *                                    (values_ptr, val_offsets_ptr, row_offsets_ptr, weight_ptr,
 *                                     out_ptr, batch_size, emb_dim, max_idx, BLOCK_SIZE)
 *   - online_best/infer.py:1029-1059 its launch from RepEncoder.forward (grid (B, 28),
 *                                    out allocated by the caller in the weight dtype)
 *   - online_best/infer.py:960-974   per-slot (values, offsets) -> flat layout (torch.cat on device)
 *   - online_best/infer.py:581-631   per-field concatenation of K cached sub-batches
 *   - baseline/infer.py:253-266      per-field clamp + nn.Embedding + segment_reduce(sum) + cat
 *
 * Conventions
 *   - Every pointer argument is a device pointer unless stated otherwise ("host" below).
 *   - Nothing here allocates device memory, synchronises the host, or throws (the one static
 *     device array of cti_ebag_forward_static is part of the loaded library). Work is
 *     enqueued on `stream` (a hipStream_t; NULL = the default stream) and runs asynchronously.
 *   - Return value: CTI_EBAG_OK (0) or a negative CTI_EBAG_E* code; the message of the last
 *     failure on the calling host thread is returned by cti_ebag_last_error().
 *   - Argument validation happens on the host before any HIP call, so argument errors are
 *     reported without touching a GPU.
 *   - Sign ids are clamped to [0, rows-1] (online_best/infer.py:823, baseline/infer.py:259);
 *     row 0 is read like any other row (no padding mask in the forward pass).
 *   - Bag (f, b) with end <= start is empty and pools to exactly 0 (sum and mean).
 *   - Accumulation is fp32; the result is rounded once to the output dtype
 *     (round-to-nearest-even for bf16/fp16).
 *   - Offsets are int64. Offsets outside [0, nnz] are clipped into that range on the device
 *     (the reference assumes well-formed offsets; clipping keeps a malformed batch from
 *     reading outside `values`).
 *   - Calls that share an output buffer or a workspace must not overlap in time.
 */
#ifndef CTI_EBAG_H
#define CTI_EBAG_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CTI_EBAG_ABI_VERSION 5

/* element types of tables and outputs */
#define CTI_EBAG_F32 0
#define CTI_EBAG_BF16 1
#define CTI_EBAG_F16 2
/* int8 row-quantised tables only (online_best/infer.py:893-942): element = q * row_scale[row] */
#define CTI_EBAG_I8 3

/* index (sign id) types */
#define CTI_EBAG_I64 0
#define CTI_EBAG_I32 1

/* pooling modes */
#define CTI_EBAG_SUM 0
#define CTI_EBAG_MEAN 1

/* status codes */
#define CTI_EBAG_OK 0
#define CTI_EBAG_EINVAL (-1)      /* bad argument (null pointer, negative size, bad enum, ...) */
#define CTI_EBAG_EUNSUPPORTED (-2) /* well-formed but outside what the library implements */
#define CTI_EBAG_EHIP (-3)        /* a HIP runtime call failed (message carries hipGetErrorString) */
#define CTI_EBAG_EWORKSPACE (-4)  /* workspace missing or smaller than cti_ebag_workspace_bytes() */

/* One field's table. `data` is a device pointer to a row-major [rows, row_stride] matrix of
 * which the first `dim` columns are used. `out_col` is the first output column of the field.
 * Several fields may share one `data` pointer (the reference's single shared nn.Embedding).
 * `row_scale` (fp32 [rows], device) is required for CTI_EBAG_I8 tables and ignored otherwise. */
typedef struct cti_ebag_table {
  const void* data;
  int64_t rows;
  int64_t row_stride; /* elements between consecutive rows, >= dim */
  int32_t dim;
  int32_t out_col;
  const float* row_scale;
} cti_ebag_table;

/* Tuning knobs of one call. Zero-initialise and set only what you need:
 *   long_threshold:  bags longer than this are not pooled by one lane group but split over all
 *                    lane groups of a wavefront (partials combined in a fixed order).
 *                    0 = default; a negative value splits every non-empty bag (used by tests).
 *                    At the default, fields of 256-byte rows (fp32 D = 64, bf16 / fp16 D = 128)
 *                    and int8 D = 128 rows take streamed tiles instead: one wavefront walks a
 *                    tile's rows in order, so every bag, whatever its length, is a sequential
 *                    fp32 sum. Conditions: no binning, nnz < 2^28 and nnz * sizeof(id) < 4 GiB,
 *                    and every table of the streamed group with a power-of-two row stride in
 *                    bytes and (rows + 1) * row stride <= 4 GiB. Otherwise those fields take the
 *                    length-ranked tiles and bags above 24 rows are split as described above.
 *   use_bins:        1 = run the device length-binning pass first: bags longer than
 *                    block_threshold are listed in the workspace and pooled by a second kernel
 *                    (one wavefront per bag, or, above split_threshold, the wavefronts of a
 *                    workgroup with partials combined through LDS in wavefront order). Needs the
 *                    workspace.
 *   block_threshold: with use_bins, the length above which a bag goes to that kernel
 *                    (0 = default, 512).
 *   split_threshold: with use_bins, listed bags up to this length are pooled by one wavefront
 *                    each (lane groups take interleaved rows); longer ones are split across the
 *                    wavefronts of a workgroup (0 = default, 192).
 * Dispatch order (no counterpart in the reference, whose Triton launch runs one program per bag).
 * A launch ends with a drain: tiles of long bags that start late run on while the rest of the GPU
 * idles. A serving loop that knows its next batch lets each call sort that batch's tiles, most
 * rows per bag first within each XCD's share, in 8 extra workgroups of the current launch; the
 * next call follows that order. Results are the same bit for bit with or without an order.
 *   tile_order:      device buffer written by an earlier call's next_order (NULL = none). An
 *                    order made for a launch of another tile count is detected on the device and
 *                    not followed.
 *   next_order:      device buffer this call fills with the order of the batch whose offsets are
 *                    next_offsets (NULL = none); it must not overlap tile_order.
 *   next_offsets:    that batch's offsets, same layout and size as `offsets` (same batch_size and
 *                    fields); only the offsets are read, while this call runs.
 *   order_bytes:     size of each order buffer, >= cti_ebag_order_bytes(batch_size, num_fields).
 * An order applies to jobs whose fields all take the same tiled row shape (one aligned row width),
 * with at most 64 fields and no binning (CTI_EBAG_EUNSUPPORTED otherwise). Calls that read or
 * write the same order buffer on different streams race.                                          */
typedef struct cti_ebag_options {
  int32_t long_threshold;
  int32_t use_bins;
  int32_t block_threshold;
  int32_t split_threshold;
  const int32_t* tile_order;
  int32_t* next_order;
  const int64_t* next_offsets;
  int64_t order_bytes;
} cti_ebag_options;

/* ABI version this library was built with (CTI_EBAG_ABI_VERSION). */
int cti_ebag_abi_version(void);

/* Message describing the last failure on this host thread ("" if none). */
const char* cti_ebag_last_error(void);

/*
 * Reference-layout entry point: a drop-in for the launch
 *   fused_all_slots_embedding_kernel[(batch_size, num_slots)](values, val_offsets, row_offsets,
 *       weight, out, batch_size, emb_dim, max_idx, BLOCK_SIZE=next_pow2(emb_dim))
 * at online_best/infer.py:1052-1059 (kernel body online_best/infer.py:805-827).
 *
 *   values      int64 [nnz]                field-major sign ids (online_best/infer.py:471)
 *   val_offsets int64 [num_slots]          start of each slot inside `values` (:473)
 *   row_offsets int64 [num_slots*(B+1)]    per-slot local bag offsets, each slot starts at 0 (:472)
 *   weight      [max_idx+1, emb_dim]       one table shared by all slots, dtype `dtype`
 *   out         [B, num_slots*emb_dim]     written in `dtype`, slot-major columns (:826)
 *   nnz         length of `values` (bounds the clipping of malformed offsets)
 * Sum pooling, fp32 accumulation, result rounded once to `dtype` (:819-827).
 */
int cti_ebag_fused_all_slots(const int64_t* values, const int64_t* val_offsets,
                             const int64_t* row_offsets, const void* weight, int32_t dtype,
                             void* out, int64_t batch_size, int32_t num_slots, int32_t emb_dim,
                             int64_t max_idx, int64_t nnz, void* stream);

/*
 * General entry point (per-field tables, global offsets, sum/mean).
 *   values        [nnz] sign ids of type `index_type`, field-major
 *   offsets       int64 [num_fields*B + 1]; bag (f, b) = values[offsets[f*B+b] : offsets[f*B+b+1]]
 *   tables        host array of num_fields descriptors (read during the call only)
 *   table_dtype   element type shared by all tables (CTI_EBAG_I8: int8 rows times each table's
 *                 row_scale, pooled as acc = fma(q, scale, acc))
 *   pooling       CTI_EBAG_SUM or CTI_EBAG_MEAN (mean of an empty bag is 0)
 *   out           [B, out_row_stride] of `out_dtype`; field f writes columns
 *                 [out_col_f, out_col_f + dim_f)
 *   workspace     device scratch of at least cti_ebag_workspace_bytes(...) bytes, 256-byte
 *                 aligned, when opts->use_bins is set (else may be NULL). Its first 16 bytes must
 *                 be zero before the first use; every call leaves the two list counters in them
 *                 (bytes 0-3 and 8-11) zero again, so one workspace serves any number of calls,
 *                 one call at a time.
 *   opts          host pointer, may be NULL (all defaults)
 * Replaces the per-field loop at baseline/infer.py:256-263 and generalises the reference
 * kernel (online_best/infer.py:805-827) to per-field tables and mean pooling.
 */
int cti_ebag_forward(const void* values, int32_t index_type, int64_t nnz, const int64_t* offsets,
                     int64_t batch_size, int32_t num_fields, const cti_ebag_table* tables,
                     int32_t table_dtype, int32_t pooling, void* out, int32_t out_dtype,
                     int64_t out_row_stride, void* workspace, int64_t workspace_bytes,
                     const cti_ebag_options* opts, void* stream);

/*
 * Allocation-free form of cti_ebag_forward. No counterpart in the reference: it is for callers
 * that cannot allocate device memory (code under HIP graph capture, tight serving loops, hosts
 * that forbid allocation). Arguments and results are cti_ebag_forward's, without the workspace:
 * the length-binning lists live in a static device array of CTI_EBAG_STATIC_WORKSPACE_BYTES
 * inside the library, one per GPU, held until the process ends. With opts->use_bins, a job whose
 * cti_ebag_workspace_bytes(batch_size, num_fields) exceeds that size (batch_size *
 * min(num_fields, 64) > 1,398,090 bags) is rejected with CTI_EBAG_EWORKSPACE before any launch.
 * Every call on one GPU shares that GPU's array: calls that overlap in time on one GPU (other
 * streams, other host threads) race and must be serialised by the caller. The first call on a
 * device looks up that device's copy and zeroes its list counters on `stream`; every call leaves
 * them zero again.
 */
#define CTI_EBAG_STATIC_WORKSPACE_BYTES (32ll << 20)
int cti_ebag_forward_static(const void* values, int32_t index_type, int64_t nnz, const int64_t* offsets,
                            int64_t batch_size, int32_t num_fields, const cti_ebag_table* tables,
                            int32_t table_dtype, int32_t pooling, void* out, int32_t out_dtype,
                            int64_t out_row_stride, const cti_ebag_options* opts, void* stream);

/* Bytes of device workspace cti_ebag_forward needs with opts->use_bins = 1
 * (256 + 24 * batch_size * min(num_fields, 64): list counters, then the field / sample and the
 * value range of each listed bag); -1 for negative arguments. */
int64_t cti_ebag_workspace_bytes(int64_t batch_size, int32_t num_fields);

/* Bytes of each dispatch-order buffer (cti_ebag_options.tile_order / next_order) for any job of
 * batch_size samples and num_fields fields (16 + 4 * batch_size * min(num_fields, 64)); -1 for
 * negative arguments. No counterpart in the reference. */
int64_t cti_ebag_order_bytes(int64_t batch_size, int32_t num_fields);

/*
 * Device packer for the reference flat layout (online_best/infer.py:960-974, and the
 * host builders :446-474 and :139-154 which produce the same three tensors):
 *   slot_values[s]  host array of num_slots device pointers, slot s has slot_nnz[s] int64 ids
 *   slot_offsets[s] host array of num_slots device pointers, each int64 [B+1], starting at 0
 *   slot_nnz        host array of num_slots counts
 * Writes flat_values int64 [sum nnz], flat_row_offsets int64 [num_slots*(B+1)],
 * val_offsets int64 [num_slots] (exclusive prefix of slot_nnz) and, if `global_offsets`
 * is not NULL, the global form int64 [num_slots*B+1]:
 *   global_offsets[s*B+b] = val_offsets[s] + row_offsets_s[b],  global_offsets[S*B] = total nnz.
 */
int cti_ebag_pack_slots(const int64_t* const* slot_values, const int64_t* const* slot_offsets,
                        const int64_t* slot_nnz, int32_t num_slots, int64_t batch_size,
                        int64_t* flat_values, int64_t* flat_row_offsets, int64_t* val_offsets,
                        int64_t* global_offsets, void* stream);

/*
 * Device merge of K flat-layout sub-batches into one, field by field in sub-batch order
 * (online_best/infer.py:581-631, online_best/infer.py:2977-3037):
 *   sub_values[k], sub_val_offsets[k], sub_row_offsets[k]   host arrays of K device pointers
 *   sub_batch[k]    host array: samples in sub-batch k;  sub_nnz[k]: length of sub_values[k]
 * Output: the flat layout of the merged batch with B = sum sub_batch[k]:
 *   flat_values int64 [sum sub_nnz], flat_row_offsets int64 [num_slots*(B+1)],
 *   val_offsets int64 [num_slots]; optional global_offsets int64 [num_slots*B+1].
 * Slot s of sub-batch k spans sub_values[k][val_offsets_k[s] : val_offsets_k[s+1]]
 * (the last slot ends at sub_nnz[k]), as at online_best/infer.py:604-606. val_offsets_k must be
 * non-decreasing within [0, sub_nnz[k]]; an entry outside that range is clamped into it (the
 * slot shrinks, nothing outside the sub-batch is read), where the reference's Python slicing
 * would wrap a negative entry.
 */
int cti_ebag_merge_batches(const int64_t* const* sub_values,
                           const int64_t* const* sub_val_offsets,
                           const int64_t* const* sub_row_offsets, const int64_t* sub_batch,
                           const int64_t* sub_nnz, int32_t num_sub, int32_t num_slots,
                           int64_t* flat_values, int64_t* flat_row_offsets, int64_t* val_offsets,
                           int64_t* global_offsets, void* stream);

/*
 * The pair merge's form of cti_ebag_merge_batches (online_best/infer.py:2977-3037, called in the
 * timed loop at :3153): the same merge, but the merged values and row offsets pass through int32
 * as the reference's `.int()` / `.long()` casts take them (:3008-3009, :3019-3020), so an id or a
 * slot-local offset of 2^31 or more wraps to its low 32 bits read as int32 there and only there.
 * val_offsets are not cast (:3021); global_offsets[s*B+b] = val_offsets[s] + the wrapped offset.
 * Arguments as for cti_ebag_merge_batches.
 */
int cti_ebag_merge_batches_int32(const int64_t* const* sub_values,
                                 const int64_t* const* sub_val_offsets,
                                 const int64_t* const* sub_row_offsets, const int64_t* sub_batch,
                                 const int64_t* sub_nnz, int32_t num_sub, int32_t num_slots,
                                 int64_t* flat_values, int64_t* flat_row_offsets, int64_t* val_offsets,
                                 int64_t* global_offsets, void* stream);

/*
 * int8 variant of the reference-layout entry point, a drop-in for the launch
 *   fused_all_slots_embedding_kernel_int8[(batch_size, num_slots)](values, val_offsets,
 *       row_offsets, weight_int8, scale, out, batch_size, emb_dim, max_idx, BLOCK_SIZE)
 * (online_best/infer.py:904-942, launched at :991-996): as cti_ebag_fused_all_slots, with
 *   weight_int8  int8 [max_idx+1, emb_dim]  and  scale  fp32 [max_idx+1];
 *   acc = fma(q, scale[row], acc) per element in element order. The reference kernel stores
 *   acc.to(tl.bfloat16) into an output of the table's dtype (:941, :989-996), so the sum is
 *   rounded to bf16 (nearest even) first and then written in `out_dtype` (fp32: exact widening;
 *   fp16: rounded again), as the reference's output holds it.
 */
int cti_ebag_fused_all_slots_int8(const int64_t* values, const int64_t* val_offsets,
                                  const int64_t* row_offsets, const int8_t* weight_int8,
                                  const float* scale, void* out, int32_t out_dtype, int64_t batch_size,
                                  int32_t num_slots, int32_t emb_dim, int64_t max_idx, int64_t nnz,
                                  void* stream);

/*
 * Reference-layout entry point for any index / offset width and table type: the launch above
 * (or its int8 form) with
 *   values       [nnz] of `index_type` (CTI_EBAG_I64 / CTI_EBAG_I32)
 *   val_offsets  [num_slots], row_offsets [num_slots*(B+1)], both of `offset_type` (I64 / I32)
 *   table_dtype  F32 / BF16 / F16, or I8 with `scale` fp32 [max_idx+1] (else ignored; I8 results
 *                are rounded to bf16 before `out_dtype`, as in cti_ebag_fused_all_slots_int8)
 *   out          [B, num_slots*emb_dim] of `out_dtype`
 * The Triton kernel specialises on the dtypes of its pointer arguments, so the reference launch
 * (online_best/infer.py:1052-1059) accepts int32 inputs the same way; the int32 forms halve the
 * input bytes a caller moves to the device (online_best/infer.py:742-779). Ids are widened and
 * clamped on the device; results equal the int64 call's bit for bit.
 */
int cti_ebag_fused_all_slots_typed(const void* values, int32_t index_type, const void* val_offsets,
                                   const void* row_offsets, int32_t offset_type, const void* weight,
                                   int32_t table_dtype, const float* scale, void* out, int32_t out_dtype,
                                   int64_t batch_size, int32_t num_slots, int32_t emb_dim, int64_t max_idx,
                                   int64_t nnz, void* stream);

/*
 * Dispatch order of a launch, made on the HOST where the batch's offsets are produced (no
 * counterpart in the reference). The reference's Triton launch runs one program per bag
 * (online_best/infer.py:1053); here a launch ends with a drain when tiles of long bags start
 * late. An order lists each XCD's tiles most rows per bag first, which removes most of it; a
 * collate or staging pass that already holds the offsets makes it at no cost to the GPU, and the
 * launch then follows it (cti_ebag_fused_all_slots_ordered; cti_ebag_forward with
 * opts->tile_order). Results are the same bit for bit with or without an order, and with an
 * order made for another batch.
 *   offsets         HOST offsets as the launch will read them, of `offset_type` (I64 / I32):
 *                   the reference layout's row_offsets [num_slots*(B+1)] (offsets_stride = B+1)
 *                   or the global offsets [num_slots*B+1] of cti_ebag_forward (offsets_stride = B)
 *   table_dtype, emb_dim   the launch's rows, one width for every slot (they fix how many bags a
 *                   tile holds)
 *   order           HOST int32 buffer of order_bytes >= cti_ebag_order_bytes(batch_size, num_slots)
 *   num_threads     host threads to use (1..256; the staging calls' persistent pool)
 * CTI_EBAG_EUNSUPPORTED for rows that take the element-wise kernel (not whole 16-byte vectors,
 * or wider than 4 KB) and for more than 64 slots. Synchronous.
 */
int cti_ebag_order_host(const void* offsets, int32_t offset_type, int64_t offsets_stride, int64_t batch_size,
                        int32_t num_slots, int32_t table_dtype, int32_t emb_dim, int32_t* order,
                        int64_t order_bytes, int32_t num_threads);

/*
 * cti_ebag_fused_all_slots_typed following a dispatch order (NULL = none): `tile_order` is a
 * DEVICE copy of what cti_ebag_order_host wrote (order_bytes bytes). An order made for a launch of
 * another tile count is detected on the device and not followed; an order for the same tile count
 * but other offsets only changes which tiles start first.
 */
int cti_ebag_fused_all_slots_ordered(const void* values, int32_t index_type, const void* val_offsets,
                                     const void* row_offsets, int32_t offset_type, const void* weight,
                                     int32_t table_dtype, const float* scale, void* out, int32_t out_dtype,
                                     int64_t batch_size, int32_t num_slots, int32_t emb_dim, int64_t max_idx,
                                     int64_t nnz, const int32_t* tile_order, int64_t order_bytes, void* stream);

/*
 * The reference-layout pooling with the encoder's input LayerNorm fused into the writer
 * (online_best/infer.py:1050-1076: the pooled block `fused_embs` [B, S*D] and
 * layernorm_forward_kernel over its rows, :829-858): out[b] = LayerNorm(pool(b)), where pool(b)
 * is the row cti_ebag_fused_all_slots_typed would write (`pooling` CTI_EBAG_SUM as in the
 * reference, or CTI_EBAG_MEAN), rounded to `dtype`, and the LayerNorm takes fp32 mean and variance
 * over the row's S*D values, y = (x - mean) * rstd * gamma + beta, rounded once to `dtype`.
 * gamma, beta: [S*D] of `param_dtype`. The pooled row is kept on chip; only the normalised row is
 * written. Covered shapes: F32 / BF16 tables and parameters, table rows of 64..1024 bytes (a
 * power of two), S <= 64, S*D*sizeof(dtype) <= 64 KiB, 16-byte aligned weight / out / gamma /
 * beta; otherwise CTI_EBAG_EUNSUPPORTED (run cti_ebag_fused_all_slots_typed and
 * cti_ebag_layernorm instead).
 */
int cti_ebag_fused_all_slots_layernorm(const void* values, int32_t index_type, const void* val_offsets,
                                       const void* row_offsets, int32_t offset_type, const void* weight,
                                       int32_t dtype, void* out, int64_t batch_size, int32_t num_slots,
                                       int32_t emb_dim, int64_t max_idx, int64_t nnz, int32_t pooling,
                                       const void* gamma, const void* beta, int32_t param_dtype, float eps,
                                       void* stream);

/*
 * Host-side compaction of sign ids for the transfer to the device (replaces the int64
 * `.to(device, non_blocking=True)` of `_flat_values` at online_best/infer.py:745-746; the comment
 * at :744 names the int32 form). `src` and `dst` are HOST pointers (dst typically pinned):
 *   dst[i] = saturate_int32(src[i]),  i < n,
 * using up to `num_threads` threads. Saturation keeps the pooled result identical to the int64
 * ids' (every table has < 2^31 rows, so clamp(saturate(v)) == clamp(v)). Synchronous.
 */
int cti_ebag_narrow_ids(const int64_t* src, int64_t n, int32_t* dst, int32_t num_threads);

/*
 * Host side of one batch's transfer (online_best/infer.py:742-779 moves each tensor with its own
 * `.to(device)`): the `n_parts` host arrays src[p] (`src_type[p]` I64 / I32, counts[p] elements)
 * are converted to `dst_type` (I32: saturating narrow as in cti_ebag_narrow_ids; I64: widened or
 * copied) into ONE contiguous region of the pinned host buffer `pinned` (part p starts at
 * cti_ebag_stage_offset(counts, n_parts, dst_type, p), 256-byte aligned), using up to
 * `num_threads` host threads, and then one hipMemcpyAsync sends the region to `device_dst` (same
 * layout) on `stream`. Returns once the copy is enqueued; `pinned` must not be rewritten until
 * the copy has run (order on `stream`). At most 8 parts.
 */
int cti_ebag_stage_copy(const void* const* src, const int32_t* src_type, const int64_t* counts,
                        int32_t n_parts, int32_t dst_type, void* pinned, int64_t pinned_bytes,
                        void* device_dst, int32_t num_threads, void* stream);

/* Byte offset of part `part` in the staging layout above (part == n_parts: total bytes); -1 for
 * bad arguments. Host pointers only. */
int64_t cti_ebag_stage_offset(const int64_t* counts, int32_t n_parts, int32_t dst_type, int32_t part);

/*
 * Row quantisation of a table to int8, quantize_embedding_int8 (online_best/infer.py:895-901) as
 * torch evaluates it on the device:
 *   m = max_j |w[r, j]| (fp32), s = max(m * RN32(1/127), 1e-8) (the division by the Python
 *   scalar 127.0 is a multiply by its fp32 reciprocal there), q[r, j] = clamp(rint(w / s), -128, 127)
 * with IEEE fp32 division and round half to even, bit for bit.
 *   weight  [rows, row_stride] of `dtype` (F32/BF16/F16), first `dim` columns used
 *   q       int8 [rows, dim] (contiguous), scale fp32 [rows]. Tables must be finite.
 */
int cti_ebag_quantize_int8(const void* weight, int32_t dtype, int64_t rows, int64_t dim, int64_t row_stride,
                           int8_t* q, float* scale, void* stream);

/*
 * Row LayerNorm over the pooled block, a drop-in for the launch
 *   layernorm_forward_kernel[(rows,)](x, y, gamma, beta, mean_out, rstd_out, eps, Row_Size=cols)
 * at online_best/infer.py:1063-1075 (kernel body online_best/infer.py:829-858):
 *   mean = sum(x)/cols, var = sum((x - mean)^2)/cols, rstd = 1/sqrt(var + eps),
 *   y = (x - mean) * rstd * gamma + beta      (fp32 arithmetic, one rounding to `dtype`)
 *   x, y      [rows, cols] contiguous, element type `dtype` (y may alias x)
 *   gamma     [cols], beta [cols], element type `param_dtype`
 *   mean_out, rstd_out   fp32 [rows] or NULL
 * y = NULL (with both mean_out and rstd_out given; gamma / beta may then be NULL) writes the
 * statistics only, the reference kernel's M_ptr / R_ptr outputs (online_best/infer.py:851-852),
 * for cti_ebag_layernorm_linear.
 * Per-row results are deterministic (fixed reduction order).
 */
int cti_ebag_layernorm(const void* x, void* y, int64_t rows, int64_t cols, int32_t dtype,
                       const void* gamma, const void* beta, int32_t param_dtype, float eps,
                       float* mean_out, float* rstd_out, void* stream);

/*
 * The input LayerNorm followed by the encoder's Linear on the matrix cores (one launch, or two
 * when K is split over a workspace, see below):
 * replaces `norm_emb = layernorm(fused_embs)` and `rep_emb = self.linear(norm_emb)` at
 * online_best/infer.py:1061-1085 (nn.Linear(28 * D, d_model), OB:951):
 *   a[m, k] = bf16( ((x[m, k] - mean[m]) * rstd[m]) * gamma[k] + beta[k] )   (as cti_ebag_layernorm
 *             computes and stores it, given the same mean / rstd)
 *   y[m, n] = sum_k a[m, k] * weight[n, k] + bias[n]   (fp32 accumulation, one rounding to y_dtype)
 *   x        bf16 [rows, cols], 16-byte aligned, cols a multiple of 8
 *   mean, rstd  fp32 [rows] (from cti_ebag_layernorm with y = NULL, or the pooling pass); with
 *            mean, rstd, gamma and beta all NULL the kernel is the plain Linear (a = x)
 *   gamma, beta  [cols], `param_dtype` F32 / BF16, 16-byte aligned
 *   weight   bf16 [out_features, cols] (nn.Linear's layout), 16-byte aligned
 *   bias     [out_features] of `bias_dtype` F32 / BF16, or NULL
 *   y        [rows, out_features] of `y_dtype` F32 / BF16, contiguous
 *   workspace  device scratch of workspace_bytes (16-byte aligned), or NULL / 0: when few rows
 *            would leave CUs idle, K is split over several workgroups per output tile, each
 *            writing fp32 partial products here, and a second launch adds the splits in split
 *            order, adds the bias and rounds once; as many splits are used as the workspace holds
 *            (up to cti_ebag_layernorm_linear_workspace_bytes(...); none without a workspace)
 * The normalised block is never written to memory. Deterministic: a given shape and workspace
 * size always takes the same splits and accumulation order (other workspace sizes may differ in
 * the last bits, within fp32 accumulation).
 */
int cti_ebag_layernorm_linear(const void* x, int64_t rows, int32_t cols, const float* mean, const float* rstd,
                              const void* gamma, const void* beta, int32_t param_dtype, const void* weight,
                              int32_t out_features, const void* bias, int32_t bias_dtype, void* y,
                              int32_t y_dtype, void* workspace, int64_t workspace_bytes, void* stream);

/* Bytes of workspace cti_ebag_layernorm_linear uses at most for this shape (0: it never splits). */
int64_t cti_ebag_layernorm_linear_workspace_bytes(int64_t rows, int32_t cols, int32_t out_features);

#ifdef __cplusplus
}
#endif

#endif /* CTI_EBAG_H */
