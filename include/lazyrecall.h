/*
 * lazyrecall.h — C ABI of liblazyrecall_hip.so, the MI355X (gfx950) implementation of
 * LazyRecall's KV-cache management hot path.
 *
 * Conventions shared by every entry point:
 *   - All tensor arguments are raw device pointers to contiguous, row-major storage that the
 *     caller owns; the library never allocates or frees them. Sizes are element/row counts.
 *   - `stream` is a hipStream_t passed as void* (NULL = the null stream). Every launch is
 *     asynchronous on that stream; nothing here synchronises the host unless stated.
 *   - Return value: LR_OK (0) on success. On failure a non-zero LR_ERR_* code is returned and
 *     lr_last_error() gives a message for the calling thread. Argument checks happen on the host
 *     before any launch, so an LR_ERR_INVALID return means nothing was enqueued.
 *   - K/V element type is given as a byte width (`elem_bytes` in {2, 4, 8}) for pure data
 *     movement, or as an LR_DTYPE_* code where arithmetic depends on it.
 *   - Index arrays read on the device (removed rows, mappings, keep indices, descriptors) are
 *     bounds-checked per row inside the kernels: an out-of-range index leaves that output row
 *     unwritten instead of touching memory outside the operands.
 *
 * Reference citations are to wrnwwrnw/code_for_iclr27 (paths relative to its root).
 */
#ifndef LAZYRECALL_H
#define LAZYRECALL_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LR_OK 0
#define LR_ERR_INVALID 1  /* bad argument; nothing enqueued */
#define LR_ERR_HIP 2      /* the HIP runtime reported an error */

#define LR_DTYPE_F32 0
#define LR_DTYPE_F64 1
#define LR_DTYPE_F16 2
#define LR_DTYPE_BF16 3

/* Message describing the last failure on the calling thread ("" if none). */
const char* lr_last_error(void);
/* ABI revision of this header; bumped whenever a signature changes. */
int lr_abi_version(void);

/* ---------------------------------------------------------------------------------------
 * Module lazy_recall._C (csrc/bindings.cpp:20-29)
 * ------------------------------------------------------------------------------------- */

/* temporal_probabilities (csrc/scoring.cu:32-66, 205-233).
 * logits [window, groups, length] of `logits_dtype` (F32/F16/BF16), projected [groups, length]
 * f32, query_positions [window] i64, key_positions [length] f32.
 * Writes probabilities [window, groups, length] f32 and output_projection [window, groups] f32. */
int lr_temporal_probabilities(const void* logits, int logits_dtype, const float* projected,
                              const int64_t* query_positions, const float* key_positions,
                              int64_t window, int64_t groups, int64_t length, float scale,
                              float* probabilities, float* output_projection, void* stream);

/* temporal_risk (csrc/scoring.cu:68-128, 235-255). Writes result [last - first] f32. */
int lr_temporal_risk(const float* probabilities, const float* output_projection,
                     const float* projected, const float* margin, int64_t window, int64_t groups,
                     int64_t length, int64_t first, int64_t last, double epsilon, float* result,
                     void* stream);

/* append (csrc/scoring.cu:130-162, 264-292). keys/values [rows, dim], positions [rows] f32,
 * new_keys/new_values [1, heads, added, dim], cumulative [heads + 1] i32.
 * Outputs: keys/values [rows + heads*added, dim], positions [rows + heads*added] f32,
 * cumulative [heads + 1] i32, lengths [heads] i32. max_length sizes the grid exactly as the
 * reference's `maximum_length` argument does. */
int lr_append(const void* keys, const void* values, const float* positions, int64_t rows,
              const void* new_keys, const void* new_values, const int32_t* cumulative,
              int64_t heads, int64_t added, int64_t dim, int elem_bytes, int64_t logical_start,
              int64_t max_length, void* out_keys, void* out_values, float* out_positions,
              int32_t* out_cumulative, int32_t* out_lengths, void* stream);

/* One decode step's append into every layer in one launch (the per-layer append calls of
 * LazyRecallCache.update, src/lazy_recall/cache.py:33-52, for all layers; no single reference
 * counterpart). Device table of `layers` rows of LR_APPEND_WORDS i64:
 *   [0] keys ptr, [1] values ptr, [2] positions ptr (f32), [3] rows, [4] cumulative ptr (i32
 *   [heads + 1]), [5] new keys ptr, [6] new values ptr ([1, heads, added, dim]), [7] logical
 *   start, [8] first output row of the layer (exclusive prefix of rows + heads * added),
 *   [9..11] 0.
 * Each layer as lr_append; outputs packed: keys/values [sum of rows + layers*heads*added, dim],
 * positions [same] f32, cumulative [layers, heads + 1] i32, lengths [layers, heads] i32.
 * max_length = the longest head of any layer. Every key/value row must be 16-byte aligned when
 * dim * elem_bytes is a multiple of 16 (the output alignment picks the copy granule). */
#define LR_APPEND_WORDS 12
int lr_append_layers(const int64_t* table, int64_t layers, int64_t heads, int64_t added,
                     int64_t dim, int elem_bytes, int64_t max_length, void* out_keys,
                     void* out_values, float* out_positions, int32_t* out_cumulative,
                     int32_t* out_lengths, void* stream);

/* lr_append_layers with the table in HOST memory (same layout, LR_APPEND_WORDS i64 per layer;
 * no single reference counterpart, like lr_append_layers): the table is read during the call
 * and its first nine words per layer travel in the launch's kernel arguments, so the call needs
 * no device copy of it and the caller may reuse the table as soon as the call returns. At most
 * 48 layers; the other arguments and the result are those of lr_append_layers. */
int lr_append_layers_host(const int64_t* host_table, int64_t layers, int64_t heads,
                          int64_t added, int64_t dim, int elem_bytes, int64_t max_length,
                          void* out_keys, void* out_values, float* out_positions,
                          int32_t* out_cumulative, int32_t* out_lengths, void* stream);

/* compact (csrc/scoring.cu:164-188, 294-314). removed [removed_count] i64, sorted, unique.
 * Outputs [rows - removed_count, dim] and positions [rows - removed_count]. */
int lr_compact(const void* keys, const void* values, const float* positions, int64_t rows,
               int64_t dim, int elem_bytes, const int64_t* removed, int64_t removed_count,
               void* out_keys, void* out_values, float* out_positions, void* stream);

/* pool (csrc/scoring.cu:190-203, 316-329). Sliding max of odd `width` inside each segment
 * [bounds[s], bounds[s+1]). bounds [segments + 1] i64 on the device; total = scores length. */
int lr_pool(const float* scores, int64_t total, const int64_t* bounds, int64_t segments,
            int64_t max_count, int64_t width, float* out, void* stream);

/* merge (csrc/recall.cu:7-28, 54-84). mapping [out_rows] i64: >=0 selects an existing row,
 * -(i+1) selects recalled row i. recalled [recalled_rows, 2, dim] (K at [i,0], V at [i,1]). */
int lr_merge(const void* keys, const void* values, const float* positions, int64_t rows,
             const void* recalled, const float* recalled_positions, int64_t recalled_rows,
             const int64_t* mapping, int64_t out_rows, int64_t dim, int elem_bytes,
             void* out_keys, void* out_values, float* out_positions, void* stream);

/* pack (csrc/recall.cu:30-47, 86-111). Gathers rows `indices` into payload [count, 2, dim]
 * and writes metadata [count, 3] i64 = (layer, heads[i], int64(positions[indices[i]])). */
int lr_pack(const void* keys, const void* values, const float* positions, int64_t rows,
            const int64_t* indices, const int64_t* heads, int64_t count, int64_t dim,
            int elem_bytes, int64_t layer, void* payload, int64_t* metadata, void* stream);

/* batch_append (csrc/batch_append.cu:8-94). `descriptors` is a DEVICE array of
 * segments x 7 i64 in the reference's layout: {keys ptr, values ptr, positions ptr,
 * source row, old length, destination row, logical position}. new_keys/new_values hold one
 * row per segment ([segments, dim]). max_rows = max over segments of (old length + 1).
 * Output rows are written at destination row .. destination row + old length. */
int lr_batch_append(const int64_t* descriptors, int64_t segments, const void* new_keys,
                    const void* new_values, int64_t dim, int elem_bytes, int64_t max_rows,
                    void* out_keys, void* out_values, float* out_positions, void* stream);

/* batch_append with the descriptors in HOST memory (the reference's host-built table before
 * its copy to the device, csrc/batch_append.cu:49-81): the table is read during the call and
 * travels in the launch's kernel arguments, so the call needs no device copy of it and the
 * caller may reuse the table as soon as the call returns. At most 64 segments (the kernel
 * argument space); the other arguments and the result are those of lr_batch_append. */
int lr_batch_append_host(const int64_t* host_descriptors, int64_t segments,
                         const void* new_keys, const void* new_values, int64_t dim,
                         int elem_bytes, int64_t max_rows, void* out_keys, void* out_values,
                         float* out_positions, void* stream);

/* All-layer pack of one eviction batch: the per-layer _C.pack calls of record_evicted
 * (src/lazy_recall/recall/transport.py:150-167, csrc/recall.cu:30-47) in one launch.
 * layer_table: DEVICE [layers, 4] i64 = (keys ptr, values ptr, positions ptr (f32), rows) per
 * layer; rows: DEVICE [count, 3] i64 = (layer, head, row within the layer). Writes payload
 * [count, 2, dim] (key row, value row; 2-byte elements) and metadata [count, 3] i64 = (layer,
 * head, int64(position)). dim * 2 a multiple of 16; payload and every key/value buffer 16-byte
 * aligned. A descriptor whose layer or row is out of range leaves its output row unwritten. */
int lr_pack_layers(const int64_t* layer_table, int64_t layers, const int64_t* rows,
                   int64_t count, int64_t dim, void* payload, int64_t* metadata, void* stream);

/* The eviction batch of a fused layout change, packed on the device from the removal sets the
 * following lr_compact_heads(_layout) call reads: LazyRecallCache.remove_positions archives
 * its removals with transport.record_evicted before compacting (src/lazy_recall/cache.py:
 * 110-112; transport.py:129-177), which needs the removals on the host. head_table as
 * lr_compact_heads (LR_HEAD_WORDS per slot, layer-major, heads_per_layer per layer); slot s
 * with segment g >= 0 removes quotas[g] positions at positions[offsets[g]...] (ascending).
 * Writes payload [*, 2, dim] (2-byte key row, value row) and metadata [*, 3] i64 = (layer,
 * head, int64(position)) in (layer, head, position) order, at most `capacity` rows; max_rows
 * bounds any one slot's removals (it sizes the grid). payload 16-byte aligned, dim * 2 a
 * multiple of 16. */
int lr_pack_heads(const int64_t* head_table, int64_t slots, int64_t heads_per_layer,
                  const int64_t* quotas, const int64_t* offsets, const int64_t* positions,
                  int64_t max_rows, int64_t dim, int64_t capacity, void* payload,
                  int64_t* metadata, void* stream);

/* Group-mean decode queries of every layer (src/lazy_recall/recall/transport.py:293-296: the
 * last decode query [Hq, d] of each layer viewed as [H, G, d] and averaged over G in f32).
 * query_table: DEVICE [layers, 2] i64 = (queries ptr, query-head stride in elements);
 * queries of `dtype` (BF16/F16/F32), dim contiguous. out f32 [layers, heads, dim]: the G values
 * summed in order, divided by G. */
int lr_group_mean_queries(const int64_t* query_table, int64_t layers, int64_t heads,
                          int64_t groups, int64_t dim, int dtype, float* out, void* stream);

/* ---------------------------------------------------------------------------------------
 * Module lazy_recall._legacy_C (csrc/cache_legacy.cu:304-308)
 * ------------------------------------------------------------------------------------- */

/* append_flattened_cache (csrc/cache_legacy.cu:13-40, 145-197). cache [rows, dim],
 * states [total_heads, new_length, dim], head_lens/cu_head_lens i32 [total_heads (+1)].
 * Output [rows + total_heads*new_length, dim]. */
int lr_append_flattened_cache(const void* cache, int64_t rows, const void* states,
                              int64_t total_heads, int64_t new_length, int64_t dim,
                              int elem_bytes, const int32_t* head_lens,
                              const int32_t* cu_head_lens, void* out, void* stream);

/* compact_flattened_kv (csrc/cache_legacy.cu:42-61, 199-242). Gathers keep_indices
 * [keep_count] i64 rows of keys/values [rows, dim] into out [keep_count, dim]. */
int lr_compact_flattened_kv(const void* keys, const void* values, int64_t rows, int64_t dim,
                            int elem_bytes, const int64_t* keep_indices, int64_t keep_count,
                            void* out_keys, void* out_values, void* stream);

/* decision_risk_scores (csrc/cache_legacy.cu:63-135, 244-302). probabilities [groups,
 * candidates] f32, values [candidates, head_dim] of values_dtype, head_outputs and gradients
 * [groups, head_dim] f32. Writes scores [candidates] f32. */
int lr_decision_risk_scores(const float* probabilities, const void* values, int values_dtype,
                            const float* head_outputs, const float* gradients, int64_t groups,
                            int64_t candidates, int64_t head_dim, double base_margin,
                            double epsilon, float* scores, void* stream);

/* ---------------------------------------------------------------------------------------
 * Module lazy_recall._host (csrc/host.cpp:5-18)
 * ------------------------------------------------------------------------------------- */

/* register_host / unregister_host (csrc/host.cpp:5-13): page-lock caller-owned host memory
 * so copies from it run asynchronously on a side stream. */
int lr_register_host(uint64_t address, uint64_t bytes);
int lr_unregister_host(uint64_t address);

/* ---------------------------------------------------------------------------------------
 * Fused audit-step entry points. These have no single reference counterpart: each replaces a
 * Python loop of reference calls (cited per function) with one or a few launches covering
 * every (layer, KV head) segment.
 * ------------------------------------------------------------------------------------- */

/* One scored segment = one (layer, KV head). Device array of `segments` rows of
 * LR_SEG_WORDS i64, written by the caller:
 *   [0] keys ptr   (bf16 [length, dim], this head's rows of the layer's flat cache)
 *   [1] values ptr (bf16 [length, dim])
 *   [2] key positions ptr (f32 [length])
 *   [3] queries ptr (bf16; group g, query w at  ptr + (g * query_group_stride + w) * dim)
 *   [4] margin gradient ptr (f32 [groups, dim], this head's rows of the pre-projection gradient)
 *   [5] length, [6] first candidate, [7] last candidate (exclusive; first < last <= length)
 *   [8] output offset of this segment's first score
 *   [9] row-stats offset (segment index * groups * window is the natural choice)
 *   [10] projected-values offset (floats; needs groups * length floats)
 *   [11] unused, must be 0 */
#define LR_SEG_WORDS 12

/* Bytes of workspace lr_score_segments needs. */
size_t lr_score_workspace_bytes(int64_t segments, int64_t groups, int64_t window,
                                int64_t projected_floats);

/* Temporal decision-risk scores of every candidate of every segment; equal to the reference's
 * per-head temporal_head_scores (src/lazy_recall/scoring.py:152-195: projected values GEMM,
 * bf16 Q.K^T, temporal_probabilities, temporal_risk, maximum over query chunks) for all heads of
 * compute_score_table (src/lazy_recall/scoring.py:218-287) at once, without materialising
 * logits or probabilities. query_positions [window] i64, margin [1] f32 (device).
 * query_group_stride is in rows of `dim` elements. scores gets sum(last - first) floats.
 * nonfinite (device i32, may be NULL) receives the number of non-finite scores, so callers can
 * refuse a table (src/lazy_recall/scoring.py:292-293) without a separate reduction.
 * stages: 0 (or 7) runs the whole scorer; otherwise a bitmask of 1 = projected values,
 * 2 = row statistics, 4 = column scores, run in that order (for per-kernel timing; each stage
 * needs the earlier ones to have run on the same workspace). With a power-of-two scale
 * (1/sqrt(dim) for dim 64 and 256) the passes skip the second bf16 rounding, which is exact
 * there; bit 8 of stages (a test hook) keeps the general form, whose scores are the same. */
int lr_score_segments(const int64_t* segment_table, int64_t segments, int64_t groups,
                      int64_t window, int64_t dim, int64_t max_length, int64_t max_candidates,
                      int64_t query_group_stride, const int64_t* query_positions,
                      const float* margin, float scale, double epsilon, void* workspace,
                      size_t workspace_bytes, float* scores, int32_t* nonfinite, int stages,
                      void* stream);

/* Test hook for the parity suite: the bf16 logits Q.K^T exactly as lr_score_segments forms them
 * (same MFMA sequence), for one segment: out [groups, window, length] bf16 (raw, unscaled). */
int lr_debug_segment_logits(const int64_t* segment_table, int64_t segment, int64_t groups,
                            int64_t window, int64_t dim, int64_t length,
                            int64_t query_group_stride, uint16_t* out, void* stream);

/* Bytes of workspace lr_select_refine needs for a table of `total` scores. */
size_t lr_select_workspace_bytes(int64_t total, int64_t segments, int64_t count);

/* Allocation-preserving Pool7 selection (src/lazy_recall/selection.py:52-88,
 * refine_arrays + transplant) on the device. raw/pooled [total] f32 score tables,
 * segment_ends [segments] i64 (cumulative ends) and position_starts [segments] i64 (device).
 * count in [1, total]. Ties at the cut go to the lower index in both bottom-k steps.
 * Outputs (device): out_values f32 [count] ascending raw scores; out_segments i64 [count];
 * out_positions i64 [count] (position_start + refined local index, transplanted);
 * quotas i64 [segments]; offsets i64 [segments + 1] (exclusive prefix of quotas);
 * removed_positions i64 [count] (each segment's refined positions, ascending, at its offset);
 * changed i64 [segments] (refined picks absent from the raw picks). */
int lr_select_refine(const float* raw, const float* pooled, int64_t total,
                     const int64_t* segment_ends, const int64_t* position_starts,
                     int64_t segments, int64_t count, void* workspace, size_t workspace_bytes,
                     float* out_values, int64_t* out_segments, int64_t* out_positions,
                     int64_t* quotas, int64_t* offsets, int64_t* removed_positions,
                     int64_t* changed, void* stream);

/* lr_select_refine in two halves, so that a caller can overlap the queue order with the
 * compaction that needs only the removal sets (src/lazy_recall/controller.py:148-158 removes
 * the first `immediate` queue entries; with immediate == count the sets are all it uses).
 * _sets: quotas, offsets, removed_positions and changed, as lr_select_refine.
 * _queue: out_values, out_segments, out_positions, as lr_select_refine; it reads what _sets
 * left in `workspace`, `quotas` and `offsets`, so it must be ordered after _sets (same stream,
 * or an event) with the same arguments, and before the workspace is reused.
 * host_info (may be NULL): host-coherent memory (lr_staging_alloc) of segments + 1 int64
 * words; _sets also writes the quotas there, and in word [segments] the i32 at `nonfinite`
 * (device, may be NULL: 0), so a host that waits for _sets reads them without a copy. */
int lr_select_refine_sets(const float* raw, const float* pooled, int64_t total,
                          const int64_t* segment_ends, const int64_t* position_starts,
                          int64_t segments, int64_t count, void* workspace,
                          size_t workspace_bytes, int64_t* quotas, int64_t* offsets,
                          int64_t* removed_positions, int64_t* changed, int64_t* host_info,
                          const int32_t* nonfinite, void* stream);
int lr_select_refine_queue(const int64_t* position_starts, int64_t total, int64_t segments,
                           int64_t count, void* workspace, size_t workspace_bytes,
                           const int64_t* quotas, const int64_t* offsets, float* out_values,
                           int64_t* out_segments, int64_t* out_positions, void* stream);

/* lr_pool followed by lr_select_refine_sets on the pooled table, in one call: controller.py:147-150
 * (pool_score_table, scoring.py:322-353, then allocation_preserving_references,
 * selection.py:52-88). The pool launch also resets the selection's counters in `workspace`,
 * which saves lr_select_refine_sets' own reset launch. raw, total, bounds [segments + 1],
 * max_count, width and pooled (output) as lr_pool; the rest as lr_select_refine_sets, whose
 * _queue half may follow with the same workspace. */
int lr_pool_select_refine_sets(const float* raw, int64_t total, const int64_t* bounds,
                               int64_t max_count, int64_t width, float* pooled,
                               const int64_t* segment_ends, const int64_t* position_starts,
                               int64_t segments, int64_t count, void* workspace,
                               size_t workspace_bytes, int64_t* quotas, int64_t* offsets,
                               int64_t* removed_positions, int64_t* changed, int64_t* host_info,
                               const int32_t* nonfinite, void* stream);

/* One head slot per (layer, KV head), LR_HEAD_WORDS i64 each (device):
 *   [0] keys ptr, [1] values ptr, [2] positions ptr (this head's first row),
 *   [3] length, [4] score-segment index or -1, [5] unused (0). */
#define LR_HEAD_WORDS 6

/* Removes every segment's `removed_positions` (from lr_select_refine) from its head and packs
 * all heads, in head-slot order, into one output [total_out_rows, dim] + positions
 * [total_out_rows] f32 (the compaction loop of src/lazy_recall/cache.py:113-178 for all layers
 * at once). max_length = largest head length. */
int lr_compact_heads(const int64_t* head_table, int64_t heads, const int64_t* quotas,
                     const int64_t* offsets, const int64_t* removed_positions, int64_t dim,
                     int elem_bytes, int64_t max_length, int64_t total_out_rows,
                     void* out_keys, void* out_values, float* out_positions, void* stream);
/* lr_compact_heads plus the compacted layers' metadata on the device, written by the same
 * launch (the per-layer rebuild of metadata.head_lens / metadata.cu_seqlens_k after a
 * compaction, src/lazy_recall/cache.py:171-177, without its host-to-device copies). The head
 * slots are layer-major with heads_per_layer heads per layer. head_lens: device i32
 * [heads] (the new length of every slot); cumulative: device i32 [layers, heads_per_layer + 1]
 * (per layer 0 then the running sum). With head_lens NULL it is lr_compact_heads. */
int lr_compact_heads_layout(const int64_t* head_table, int64_t heads, const int64_t* quotas,
                            const int64_t* offsets, const int64_t* removed_positions,
                            int64_t dim, int elem_bytes, int64_t max_length,
                            int64_t total_out_rows, void* out_keys, void* out_values,
                            float* out_positions, int64_t heads_per_layer, int32_t* head_lens,
                            int32_t* cumulative, void* stream);

/* The lazy eviction queue (src/lazy_recall/controller.py:140-159 keeps references[immediate:]
 * after removing the first `immediate`; controller.py:57-70 evict_prefix removes the next
 * batches). State: the selection's per-segment position-sorted picks (quotas, offsets,
 * removed_positions of lr_select_refine) and, per pick, its queue slot `rank` (device i32
 * [count], laid out like removed_positions).
 * lr_queue_index fills `rank` from the queue order (queue_segments/queue_positions [count] i64,
 * lr_select_refine_queue's out_segments/out_positions); every entry is written.
 * lr_queue_evict_plan plans the removal of queue slots [begin, end), given that slots
 * [0, begin) are already removed: per segment s, batch_quotas[s] = its slots in the range and
 * batch_positions[offsets[s] ...] = their positions ascending, each minus the number of slots
 * of s removed earlier at a lower position (the searchsorted(removed_at_audit, positions)
 * remap). (batch_quotas, offsets, batch_positions) is then what lr_compact_heads takes.
 * host_quotas (may be NULL): host-coherent memory (lr_staging_alloc) of `segments` words that
 * also receives batch_quotas. */
int lr_queue_index(const int64_t* queue_segments, const int64_t* queue_positions, int64_t count,
                   const int64_t* quotas, const int64_t* offsets,
                   const int64_t* removed_positions, int64_t segments, int32_t* rank,
                   void* stream);
int lr_queue_evict_plan(const int64_t* quotas, const int64_t* offsets,
                        const int64_t* removed_positions, const int32_t* rank, int64_t segments,
                        int64_t begin, int64_t end, int64_t* batch_quotas,
                        int64_t* batch_positions, int64_t* host_quotas, void* stream);

/* Reinsertion of recalled rows into every layer at once (insert_payload, src/lazy_recall/
 * cache.py:201-253, with merge_plan, recall/planning.py:34-52, and merge, csrc/recall.cu:7-28;
 * no single reference counterpart). Per (layer, KV head) slot, its resident rows (positions
 * ascending, as the cache keeps them) and its recalled rows (any order) merge into one head
 * ordered by position, all heads packed in slot order into one output. Device table of `slots`
 * rows of LR_REINSERT_WORDS i64 (written by the caller):
 *   [0] keys ptr, [1] values ptr, [2] positions ptr (f32) of the head's first resident row,
 *   [3] resident rows, [4] first entry of the head's run (exclusive prefix of [5]), [5] recalled
 *   rows of the head (at most LR_REINSERT_MAX_PER_HEAD), [6] first output row of the merged
 *   head, [7] 0.
 * lr_reinsert_plan: grouped = DEVICE i64 [2 * count]: the recalled positions grouped by slot
 * (slot s's run at [4] of its row, any order within the run), then at [count + j] the index in
 * the payload of grouped entry j. Sorts each run by position and finds each entry's output
 * row. workspace: device i64 [3 * count]. recalled_rows [count] i64: the row of each payload
 * entry within its merged head. flag (device i32, zeroed by the caller): bit 0 = a recalled
 * position equals a resident or another recalled one of its head (merge_plan's "duplicate
 * physical KV identities"), bit 3 = a slot with more than LR_REINSERT_MAX_PER_HEAD rows.
 * lr_reinsert_resident: the resident rows of every slot (needs only the plan: may run while
 * the payload is still being copied in). max_length = longest resident run.
 * lr_reinsert_recalled: the recalled rows, from payload [count, 2, dim] (K at [i, 0], V at
 * [i, 1]). */
#define LR_REINSERT_WORDS 8
#define LR_REINSERT_MAX_PER_HEAD 4096
int lr_reinsert_plan(const int64_t* table, int64_t slots, const int64_t* grouped, int64_t count,
                     int64_t* workspace, int64_t* recalled_rows, int32_t* flag, void* stream);
/* Device grouping for a reinsertion whose identities are in device memory: the host's
 * grouping and counting of reinsert_prepare (merge_plan's per-head runs, src/lazy_recall/
 * recall/planning.py:34-52) done by three launches on `stream`, so that the host never walks
 * the identities. table: DEVICE, LR_REINSERT_WORDS per slot with words [0..3] filled and [4..7]
 * zero; metadata: DEVICE i64 [count, 3] (layer, head, position). Fills table words [4] (first
 * entry of the slot's run), [5] (recalled rows of the slot) and [6] (first output row), and
 * grouped = DEVICE i64 [2 * count] as lr_reinsert_plan takes it (runs in any order inside).
 * host_counts (host-coherent, lr_staging_alloc, or NULL) receives each slot's recalled rows
 * for the host's layout. flag as lr_reinsert_plan's, plus bit 2: an identity outside the
 * layers, heads or [0, 2^31) (left out of every run). */
int lr_reinsert_group(int64_t* table, int64_t slots, int64_t heads, const int64_t* metadata,
                      int64_t count, int64_t* grouped, int64_t* host_counts, int32_t* flag,
                      void* stream);
/* lr_reinsert_plan plus the merged layers' metadata on the device, written by the same
 * launch (LazyRecallCache.insert_payload's replace_head_lens, src/lazy_recall/cache.py:246,
 * without its host-to-device copies): head_lens i32 [slots] and cumulative i32
 * [layers, heads_per_layer + 1], as lr_compact_heads_layout. With head_lens NULL it is
 * lr_reinsert_plan; with it, the launch also runs when count is 0. */
int lr_reinsert_plan_layout(const int64_t* table, int64_t slots, const int64_t* grouped,
                            int64_t count, int64_t* workspace, int64_t* recalled_rows,
                            int32_t* flag, int64_t heads_per_layer, int32_t* head_lens,
                            int32_t* cumulative, void* stream);
int lr_reinsert_resident(const int64_t* table, int64_t slots, const int64_t* workspace,
                         int64_t count, int64_t max_length, int64_t dim, int elem_bytes,
                         int64_t out_rows, void* out_keys, void* out_values, float* out_positions,
                         void* stream);
int lr_reinsert_recalled(const int64_t* workspace, int64_t count, const void* payload,
                         int64_t dim, int elem_bytes, int64_t out_rows, void* out_keys,
                         void* out_values, float* out_positions, void* stream);

/* Staging of the fused step's metadata block (no reference counterpart: the reference copies
 * each per-layer index list to the device with its own blocking copy). lr_staging_alloc gives
 * `bytes` of pinned, host-coherent memory that kernels may read directly; lr_staging_free
 * releases it (no kernel may still read it). lr_copy_words copies `words` 8-byte words from such
 * memory (or from device memory) to device memory, or from device memory to such host memory,
 * with a kernel on `stream`, so a small copy between two kernels needs no copy-engine round
 * trip. */
int lr_staging_alloc(size_t bytes, void** host);
int lr_staging_free(void* host);
int lr_copy_words(const int64_t* source, int64_t* destination, int64_t words, void* stream);

/* Calibration copy (no reference counterpart): copies `bytes` (a multiple of 16; both buffers
 * 16-byte aligned device memory) with the nontemporal 16-byte loads and stores that the
 * all-layer row kernels use, on `stream`. Timed on a copy far beyond the caches, it gives the
 * practical read+write ceiling those kernels are measured against. */
int lr_stream_copy(const void* source, void* destination, int64_t bytes, void* stream);

/* Device-resident query history (replaces the per-layer deques and the per-audit torch.cat of
 * src/lazy_recall/history.py:21-38,51-63). `ring` is [layers, heads, 2 * window, dim] elements
 * of elem_bytes (2 or 4) and ring_positions [2 * window] i64, both device memory. Writes query l
 * (layer_queries[l], device, [heads, dim] contiguous) to rows `slot` and `slot + window` of every
 * head of layer l and `position` to ring_positions[slot] and [slot + window], with one launch per
 * LR_HISTORY_MAX_LAYERS layers. Appending the k-th query (0-based) at slot k mod window keeps the
 * last min(n, window) queries in rows [s, s + min(n, window)), s = n mod window once n >= window
 * (else 0), oldest first: a strided [heads, n, dim] view the fused scorer reads in place. */
#define LR_HISTORY_MAX_LAYERS 128
int lr_history_append(const void* const* layer_queries, int64_t layers, int64_t heads,
                      int64_t dim, int elem_bytes, int64_t window, int64_t slot, void* ring,
                      int64_t position, int64_t* ring_positions, void* stream);

/* ---------------------------------------------------------------------------------------
 * Decode/prefill attention over the packed ragged layout
 * ------------------------------------------------------------------------------------- */

/* packed_attention (src/lazy_recall/attention.py:15-35; its flash_attn_varlen_func call with
 * causal=True, softmax_scale = dim^-0.5, one KV head per segment). Segment s = b * kv_heads + h
 * owns key/value rows [cu_seqlens_k[s], cu_seqlens_k[s+1]) (device i32 [batch*kv_heads + 1]) of
 * keys/values [key_rows, dim]. queries are [batch, kv_heads*groups, length, dim] elements with
 * the given element strides (dim contiguous); query head h*groups + g belongs to segment h.
 * Causal masking is aligned to the segment end (query i sees keys j <= i + n_s - length); a row
 * with no visible key is zero. out is [batch, length, kv_heads*groups, dim] contiguous, of the
 * input dtype (LR_DTYPE_BF16 or LR_DTYPE_F16); dim in {64, 128, 256}. max_keys bounds every
 * segment's key count (keys past it are not read). workspace: device scratch of at least
 * lr_packed_attention_workspace_bytes(...) bytes (0 when every segment fits one block of keys),
 * 256-byte aligned, no initial contents required; calls that overlap in time need their own.
 * Two launches when a segment spans several key blocks (blocks, then their merge). */
size_t lr_packed_attention_workspace_bytes(int64_t segments, int64_t groups, int64_t length,
                                           int64_t max_keys, int64_t dim);
int lr_packed_attention(const void* queries, int64_t q_batch_stride, int64_t q_head_stride,
                        int64_t q_query_stride, const void* keys, const void* values,
                        int64_t key_rows, const int32_t* cu_seqlens_k, int64_t batch,
                        int64_t kv_heads, int64_t groups, int64_t length, int64_t dim, int dtype,
                        int64_t max_keys, float scale, void* out, void* workspace,
                        size_t workspace_size, void* stream);
/* Decode attention over each segment's cached rows plus one pending row: the step's own new
 * token of each (request, KV head), not yet appended (no reference counterpart as an entry
 * point: the reference appends inside each layer's forward, src/lazy_recall/attention.py:63
 * -> cache.py:33-52, and attends over the appended cache). The pending row is key n of its
 * segment (n = the cached rows), exactly where the append would put it, so the output equals
 * lr_packed_attention over the appended cache, bit for bit; a decode step can then append
 * every layer's tokens afterwards in one lr_append_layers launch. One query per segment
 * (length 1); pending_keys / pending_values: [batch * kv_heads, dim] in the queries' dtype
 * (segment s = request b * kv_heads + head h), 16-byte aligned. The workspace is sized by
 * lr_packed_attention_pending_workspace_bytes; max_keys = the longest cached segment. */
size_t lr_packed_attention_pending_workspace_bytes(int64_t segments, int64_t groups,
                                                   int64_t max_keys, int64_t dim);
int lr_packed_attention_pending(const void* queries, int64_t q_batch_stride,
                                int64_t q_head_stride, int64_t q_query_stride, const void* keys,
                                const void* values, int64_t key_rows,
                                const int32_t* cu_seqlens_k, int64_t batch, int64_t kv_heads,
                                int64_t groups, int64_t dim, int dtype, int64_t max_keys,
                                float scale, const void* pending_keys,
                                const void* pending_values, void* out, void* workspace,
                                size_t workspace_size, void* stream);

/* Allocation-free packed attention. No counterpart in the reference: it is for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc). Same arguments, kernels and results as lr_packed_attention, without
 * the workspace: the partial states live in one fixed array per device of
 * lr_packed_attention_scratch_bytes() bytes (16 MiB), held from the library's first use on that
 * device until the process ends. The call allocates and frees nothing. A call whose
 * lr_packed_attention_workspace_bytes(...) exceeds that size returns LR_ERR_INVALID with a
 * message naming both sizes, before anything is enqueued. Every call on one device shares that
 * device's array and leaves its contents behind (none are needed at the next call): two calls
 * that can overlap in time on one device (different streams without an order between them)
 * race on it. The device is the one that owns `stream` (the current device for NULL). */
size_t lr_packed_attention_scratch_bytes(void);
int lr_packed_attention_noalloc(const void* queries, int64_t q_batch_stride,
                                int64_t q_head_stride, int64_t q_query_stride, const void* keys,
                                const void* values, int64_t key_rows,
                                const int32_t* cu_seqlens_k, int64_t batch, int64_t kv_heads,
                                int64_t groups, int64_t length, int64_t dim, int dtype,
                                int64_t max_keys, float scale, void* out, void* stream);

/* ---------------------------------------------------------------------------------------
 * Audit vector-Jacobian helpers (the margin objective and its gradients)
 * ------------------------------------------------------------------------------------- */

/* last_token_logits_float32 (src/lazy_recall/_core/scoring.py:34-52): out[r, v] =
 * sum_d hidden[r, d] * weight[v, d] (+ bias[v]) in f32. hidden [rows, dim] f32, weight
 * [vocab, dim] and bias [vocab] (may be NULL) of `dtype` (F32/F16/BF16), out [rows, vocab] f32.
 * dim a multiple of 8, at most 8192; weight 16-byte aligned. */
int lr_head_logits(const float* hidden, int64_t rows, const void* weight, const void* bias,
                   int64_t vocab, int64_t dim, int dtype, float* out, void* stream);

/* one_vs_rest_margin / row_margins (src/lazy_recall/_core/scoring.py:27-31,
 * batch_audit.py:11-15): per logits row r ([rows, vocab] f32), the target t = targets[r]
 * (device i64, or NULL: the first argmax), the competitor max M = max_{v != t} l_v and sum
 * S = sum_{v != t} exp(l_v - M); margins[r] = l_t - (M + log S), stats[r] = (M, S). targets_out
 * (may be NULL) receives t. workspace: device scratch of lr_margin_stats_workspace_bytes bytes,
 * 16-byte aligned, no initial contents. */
size_t lr_margin_stats_workspace_bytes(int64_t rows, int64_t vocab);
int lr_margin_stats(const float* logits, int64_t rows, int64_t vocab, const int64_t* targets,
                    int64_t* targets_out, float* margins, float* stats, void* workspace,
                    size_t workspace_size, void* stream);

/* Workspace of lr_hidden_gradient / lr_pre_gradient (device, 16-byte aligned, no contents). */
size_t lr_row_sum_workspace_bytes(int64_t rows, int64_t vocab, int64_t dim);

/* one_vs_rest_hidden_gradient / row_hidden_gradients (src/lazy_recall/_core/scoring.py:54-76,
 * batch_audit.py:18-24): out[r, :] = (weight[t_r, :] - sum_v p[r, v] * weight[v, :]) * due[r],
 * p[r] the softmax of row r's logits with the target excluded (p = exp(l - M) / S from
 * lr_margin_stats' stats, 0 at t_r). due (may be NULL: 1) [rows] f32, out [rows, dim] f32. */
int lr_hidden_gradient(const float* logits, const float* stats, const int64_t* targets,
                       int64_t rows, const void* weight, int64_t vocab, int64_t dim, int dtype,
                       const float* due, float* out, void* workspace, size_t workspace_size,
                       void* stream);

/* Pre-projection margin gradient of one layer (src/lazy_recall/scoring.py:228-237):
 * out[q] = sum_h post_gradient[h] * o_weight[h, q] (* gate[q] when gate is not NULL).
 * post_gradient [hidden] f32, o_weight [hidden, width] of `dtype`, gate [width] f32. */
int lr_pre_gradient(const float* post_gradient, const void* o_weight, int64_t hidden,
                    int64_t width, int dtype, const float* gate, float* out, void* workspace,
                    size_t workspace_size, void* stream);

/* The pre-projection gradients of several layers in one launch pair (the loop of
 * src/lazy_recall/scoring.py:218-237 over layers; no single reference counterpart). layer_table:
 * DEVICE [layers, 4] i64 = (o_weight [hidden, width] of `dtype`, post_gradient [hidden] f32,
 * gate [width] f32 or 0, out [width] f32) per layer, all valid device addresses, weights 16-byte
 * aligned; every layer shares hidden, width and dtype. */
size_t lr_pre_gradient_layers_workspace_bytes(int64_t layers, int64_t hidden, int64_t width);
int lr_pre_gradient_layers(const int64_t* layer_table, int64_t layers, int64_t hidden,
                           int64_t width, int dtype, void* workspace, size_t workspace_size,
                           void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LAZYRECALL_H */
