/*
 * kvcompress_mi355x.h -- C ABI of the MI355X TriAttention KV-compression path.
 *
 * Path: paged-K trigonometric scoring -> per-head normalisation and
 * cross-layer aggregation -> per-sequence keep-set selection -> K/V
 * compaction with block-table rewrite and page release.
 *
 * Conventions shared by every entry point:
 *   - All pointers are device pointers unless the parameter name ends in
 *     "_host".  Nothing is allocated and nothing is freed; scratch memory is
 *     passed in by the caller (sizes come from the *_workspace_bytes queries).
 *   - Work is enqueued on `stream` (a hipStream_t; NULL = default stream) and
 *     never synchronised.
 *   - Return value: 0 on success, KVC_EINVAL for rejected arguments, or a
 *     positive hipError_t from the launch.  kvc_last_error() returns the
 *     message of the last failure on the calling thread.
 *   - Caches use the reference layout [num_pages][128][kv_heads][head_dim]
 *     (bf16 or fp16) with contiguous inner dimensions and a page stride
 *     >= 128*kv_heads*head_dim elements (pkg/provider.py:1201-1230).
 *     Per-layer caches are named by a device table of base addresses.
 *   - Token blocks are 128 tokens (pkg/config.py:18, ASCEND_BLOCK_SIZE).
 *   - Block tables are int64 (source_block_ids_device, pkg/methods/base.py:74).
 *     A batch of sequences uses ragged tables: sequence b owns
 *     block_ids[block_offsets[b] .. block_offsets[b+1]).
 *
 * Citations are to the reference repository vLLM-HUST/vllm-ascend-kvcompress-hust
 * v0.10.0 with tri/ = src/vllm_ascend_kvcompress/methods/triattention/ and
 * pkg/ = src/vllm_ascend_kvcompress/.
 */
#ifndef KVCOMPRESS_MI355X_H
#define KVCOMPRESS_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* kvc_stream_t; /* hipStream_t */

#define KVC_ABI_VERSION 2
#define KVC_BLOCK_SIZE 128
#define KVC_EINVAL (-22)

enum kvc_dtype { KVC_DTYPE_BF16 = 0, KVC_DTYPE_FP16 = 1, KVC_DTYPE_FP32 = 2 /* query statistics only */ };
enum kvc_rope_style { KVC_ROPE_HALF = 0, KVC_ROPE_INTERLEAVED = 1 };
enum kvc_policy { KVC_POLICY_GLOBAL = 0, KVC_POLICY_V3 = 1 };
enum kvc_layer_aggregation { KVC_LAYER_MEAN = 0, KVC_LAYER_MAX = 1 };
enum kvc_raw_layout { KVC_RAW_TOKEN_MAJOR = 0, KVC_RAW_HEAD_MAJOR = 1 };

/* Flags of kvc_aggregate. */
#define KVC_AGG_ACCUMULATE 1u /* combine with the existing aggregate instead of overwriting it */
#define KVC_AGG_FINALIZE 2u   /* divide by the layer count (mean mode) and sanitise NaN/inf */
#define KVC_AGG_RSQRT 4u      /* (s-mean)*rsqrt(max(var,1e-6)) instead of (s-mean)/sqrt(max(var,1e-6)) */
#define KVC_COMPACT_LAYER_MAJOR 0      /* kvc_compact order: planned copy one layer at a time */
#define KVC_COMPACT_LAYERS_INTERLEAVED 1 /* kvc_compact order: planned copy with all layers interleaved */

/* ABI version and last error message of the calling thread. No counterpart in
 * the reference (it is a pure-Python plugin). */
int kvc_abi_version(void);
const char* kvc_last_error(void);

/* ---------------------------------------------------------------- phases -- */

/* Mean future-position phase coefficients, evaluated directly:
 *   phase_cos[b][l][f] = mean_o cos((offsets[o] + round_starts[b]) * omega[l][f])
 *   phase_sin[b][l][f] = mean_o sin((offsets[o] + round_starts[b]) * omega[l][f])
 * Replaces the torch path's phase evaluation inside score_post_rope_keys
 * (tri/scoring.py:77-80) for every sequence and scoring layer at once. */
int kvc_mean_phases(kvc_stream_t stream, int n_seq, int n_layers, int n_freq,
                    const int64_t* round_starts, const float* offsets, int n_offsets,
                    const float* omega, float* phase_cos, float* phase_sin);

/* Angle-addition form of the reference's device path:
 *   phase_cos = cos(rs*omega)*offset_cos_mean - sin(rs*omega)*offset_sin_mean
 *   phase_sin = sin(rs*omega)*offset_cos_mean + cos(rs*omega)*offset_sin_mean
 * Replaces prepare_mean_phase_coefficients (tri/kernels.py:50-122). */
int kvc_shift_mean_phases(kvc_stream_t stream, int n_values, int64_t round_start,
                          const float* omega, const float* offset_cos_mean,
                          const float* offset_sin_mean, float* phase_cos, float* phase_sin);

/* --------------------------------------------------------------- scoring -- */

/* Bytes of scratch kvc_score_paged needs for this shape. */
size_t kvc_score_workspace_bytes(int n_layers, int kv_heads, int head_dim, int rotary_dim,
                                 int qpk, int n_seq, int max_seq_len);

/* Raw-score layout that kvc_score_paged writes fastest for this shape:
 * KVC_RAW_HEAD_MAJOR ([layer][head][token], raw_token_stride 1; the matrix-core
 * scorer stores four consecutive tokens of a head per lane) or
 * KVC_RAW_TOKEN_MAJOR ([layer][token][head], raw_head_stride 1; the vector
 * scorer's lanes of one token span every head).  kvc_score_paged and
 * kvc_aggregate accept either layout; this only names the faster one.
 * Returns KVC_EINVAL for a shape kvc_score_paged rejects.  The reference keeps
 * [kv_heads][qpk][max_len] per scoring layer (tri/method.py:232-240) and has
 * no such query. */
int kvc_score_raw_layout(int dtype, int rope_style, int kv_heads, int head_dim, int rotary_dim,
                         int qpk);

/* Raw TriAttention scores of every cached token against the calibrated query
 * centres (tri/scoring.py:23-120, device form tri/kernels.py:125-317):
 *   score[l][b][t][h*qpk+g] = sum_f a*((qr*kr+qi*ki)*c_f - (qi*kr-qr*ki)*s_f)
 *                           + sum_f a*extra*|k_f| + sum_p q_pass*k_pass
 * for the n_layers scoring layers, all sequences of the batch, reading K once
 * per KV head through the block tables (token t of sequence b lives in page
 * block_ids[block_offsets[b] + t/128], row t%128).
 *
 * Calibration inputs are per scoring layer, grouped by KV head, float32:
 *   q_real, q_imag, freq_scale (= sqrt(freq_scale_sq)), extra_coef
 *   (= q_abs_mean - sqrt(q_real^2+q_imag^2+1e-8)): [n_layers][kv_heads][qpk][F]
 *   q_pass: [n_layers][kv_heads][qpk][head_dim-rotary_dim], NULL when full RoPE.
 * phase_cos/phase_sin: [n_seq][n_layers][F] with sequence stride
 * phase_seq_stride elements (0 = one table shared by all sequences).
 * Output element (l, b, t, q) is written at
 *   raw[l*raw_layer_stride + (token_offsets[b]+t)*raw_token_stride + q*raw_head_stride].
 * The workspace also receives per-tile float64 partial sums used by
 * kvc_head_stats; it must stay untouched until that call. */
int kvc_score_paged(kvc_stream_t stream, int dtype, int n_layers, const uint64_t* k_layer_ptrs,
                    int64_t num_pages, int64_t page_stride, int kv_heads, int head_dim,
                    int rotary_dim, int qpk, int rope_style, int n_seq, int max_seq_len,
                    const int32_t* seq_lens, const int64_t* token_offsets,
                    const int64_t* block_offsets, const int64_t* block_ids, const float* q_real,
                    const float* q_imag, const float* freq_scale, const float* extra_coef,
                    const float* q_pass, const float* phase_cos, const float* phase_sin,
                    int64_t phase_seq_stride, float* raw, int64_t raw_layer_stride,
                    int64_t raw_token_stride, int64_t raw_head_stride, void* workspace,
                    size_t workspace_bytes);

/* Per-offset phase table for score_aggregation "max":
 *   phase_cos[b][l][o][f] = cos((offsets[o] + round_starts[b]) * omega[l][f])
 *   phase_sin[b][l][o][f] = sin((offsets[o] + round_starts[b]) * omega[l][f])
 * with the argument formed in float32 as the torch path does and the cosine
 * and sine rounded once from double.  Replaces the phases of the max branch of
 * score_post_rope_keys (tri/scoring.py:77,84-91) for every sequence and
 * scoring layer at once. */
int kvc_offset_phases(kvc_stream_t stream, int n_seq, int n_layers, int n_freq,
                      const int64_t* round_starts, const float* offsets, int n_offsets,
                      const float* omega, float* phase_cos, float* phase_sin);

/* Bytes of scratch kvc_score_paged_max needs for this shape and offset count
 * (at least kvc_score_workspace_bytes of the same shape, so kvc_head_stats
 * accepts the same workspace). 0 for an unsupported shape. */
size_t kvc_score_max_workspace_bytes(int n_layers, int kv_heads, int head_dim, int rotary_dim,
                                     int qpk, int n_seq, int max_seq_len, int n_offsets);

/* Raw scores with the rotary term maximised over the future offsets instead of
 * averaged: score_aggregation="max" of score_post_rope_keys
 * (tri/scoring.py:84-97), which the reference runs through its torch fallback
 * (tri/method.py:348-431):
 *   score[l][b][t][h*qpk+g] = max_o sum_f a*((qr*kr+qi*ki)*cos_of - (qi*kr-qr*ki)*sin_of)
 *                           + sum_f a*extra*|k_f| + sum_p q_pass*k_pass
 * Arguments as kvc_score_paged except offset_cos/offset_sin: the
 * kvc_offset_phases tables [n_seq][n_layers][n_offsets][F], sequence stride
 * phase_seq_stride elements (0 = one table shared by all sequences), at most
 * 32 offsets.  Shapes as kvc_score_paged (bf16 or fp16); the matrix-core
 * scorer serves head_dim 64, 128 or 256 with rotary_dim/2 a multiple of 32, a
 * vector-ALU scorer the rest (KVC_EINVAL when one query head's per-offset
 * weights exceed 64 KB of LDS).  Partial sums for kvc_head_stats land where
 * kvc_score_paged leaves them. */
int kvc_score_paged_max(kvc_stream_t stream, int dtype, int n_layers, const uint64_t* k_layer_ptrs,
                        int64_t num_pages, int64_t page_stride, int kv_heads, int head_dim,
                        int rotary_dim, int qpk, int rope_style, int n_seq, int max_seq_len,
                        const int32_t* seq_lens, const int64_t* token_offsets,
                        const int64_t* block_offsets, const int64_t* block_ids, const float* q_real,
                        const float* q_imag, const float* freq_scale, const float* extra_coef,
                        const float* q_pass, const float* offset_cos, const float* offset_sin,
                        int n_offsets, int64_t phase_seq_stride, float* raw,
                        int64_t raw_layer_stride, int64_t raw_token_stride,
                        int64_t raw_head_stride, void* workspace, size_t workspace_bytes);

/* Population mean and variance of every query head's raw scores over the
 * sequence's tokens, from the partial sums kvc_score_paged left in the
 * workspace (torch.var_mean(raw, dim=-1, correction=0), tri/method.py:379-381,423).
 * mean/var: float32 [n_layers][n_seq][kv_heads*qpk]. Same shape arguments as
 * the kvc_score_paged call that filled the workspace. */
int kvc_head_stats(kvc_stream_t stream, int n_layers, int kv_heads, int head_dim, int rotary_dim,
                   int qpk, int n_seq, int max_seq_len, const int32_t* seq_lens,
                   const void* workspace, size_t workspace_bytes, float* mean, float* var);

/* kvc_score_paged followed by kvc_head_stats, with the scorer's scratch (folded
 * weights and per-tile partial sums) in a static 64 MiB device array that the
 * library holds on every device it runs on until the process ends, instead of
 * a caller workspace.  No counterpart in the reference: it is for callers that
 * cannot allocate device memory (code under HIP graph capture, serving loops
 * that forbid allocation).  It allocates and frees nothing.  Arguments as
 * kvc_score_paged without the workspace, plus kvc_head_stats's mean/var
 * outputs; the results equal those two calls'.  Returns KVC_EINVAL when the
 * batch needs more scratch than 64 MiB (kvc_score_workspace_bytes of the same
 * shape; e.g. 6 scoring layers x 16 sequences of 16384 tokens x 40 query heads
 * need 7 MiB) and when `stream` does not belong to the current device.  Every
 * call on a device shares that device's array: calls that overlap in time on
 * one device (concurrent streams, several threads) race and must be
 * serialised by the caller. */
int kvc_score_paged_noalloc(kvc_stream_t stream, int dtype, int n_layers, const uint64_t* k_layer_ptrs,
                            int64_t num_pages, int64_t page_stride, int kv_heads, int head_dim,
                            int rotary_dim, int qpk, int rope_style, int n_seq, int max_seq_len,
                            const int32_t* seq_lens, const int64_t* token_offsets,
                            const int64_t* block_offsets, const int64_t* block_ids, const float* q_real,
                            const float* q_imag, const float* freq_scale, const float* extra_coef,
                            const float* q_pass, const float* phase_cos, const float* phase_sin,
                            int64_t phase_seq_stride, float* raw, int64_t raw_layer_stride,
                            int64_t raw_token_stride, int64_t raw_head_stride, float* mean, float* var);

/* Normalise, take the max over query heads and combine across layers
 * (normalize_head_scores + _aggregate_torch, tri/scoring.py:123-128,
 * tri/method.py:477-503; device form tri/kernels.py:365-437; layer mean and
 * nan_to_num tri/method.py:463-467):
 *   z = (raw - mean) / sqrt(max(var, 1e-6))       per (layer, seq, head, token)
 *   layer_score = max_h z                          (NaN-propagating)
 *   agg = layer_score[0] (+ or max) layer_score[1] ... in layer order
 * flags: KVC_AGG_ACCUMULATE combines layer 0 with the existing agg contents;
 * KVC_AGG_FINALIZE divides by n_layers (mean mode) and maps NaN->-inf,
 * +inf->1e30; KVC_AGG_RSQRT uses the reference device kernel's rsqrt form.
 * mean/var addressed as [l*stats_layer_stride + b*stats_seq_stride + h].
 * agg element (b, t) lives at agg[token_offsets[b] + t]. */
int kvc_aggregate(kvc_stream_t stream, int n_layers, int n_heads, int n_seq, int max_seq_len,
                  const int32_t* seq_lens, const int64_t* token_offsets, const float* raw,
                  int64_t raw_layer_stride, int64_t raw_token_stride, int64_t raw_head_stride,
                  const float* mean, const float* var, int64_t stats_layer_stride,
                  int64_t stats_seq_stride, int layer_aggregation, unsigned flags, float* agg);

/* Tensor-parallel halves of kvc_aggregate (the reference's TP path,
 * tri/method.py:316-322,447-461 with _aggregate_torch's defer_tp_reduce,
 * :477-503).  A rank holding a shard of the KV heads scores and normalises its
 * own query heads, writes each scoring layer's head maximum
 *   layer_scores[l*layer_stride + token_offsets[b] + t] = max_h z   (NaN-propagating)
 * with kvc_layer_head_max (flags: KVC_AGG_RSQRT only), the ranks reduce
 * layer_scores with an elementwise MAX (all_reduce(MAX) over the TP group; not
 * part of this library), and kvc_combine_layer_scores turns the reduced layer
 * scores into the aggregate: layers combined in layer order (copy, then + or
 * max), then KVC_AGG_FINALIZE's division and NaN/inf mapping if set.  With
 * every head on one rank the result equals kvc_aggregate's bit for bit. */
int kvc_layer_head_max(kvc_stream_t stream, int n_layers, int n_heads, int n_seq, int max_seq_len,
                       const int32_t* seq_lens, const int64_t* token_offsets, const float* raw,
                       int64_t raw_layer_stride, int64_t raw_token_stride, int64_t raw_head_stride,
                       const float* mean, const float* var, int64_t stats_layer_stride,
                       int64_t stats_seq_stride, unsigned flags, float* layer_scores,
                       int64_t layer_stride);
int kvc_combine_layer_scores(kvc_stream_t stream, int n_layers, int64_t n_tokens, const float* layer_scores,
                             int64_t layer_stride, int layer_aggregation, unsigned flags, float* agg);

/* ------------------------------------------------------------- selection -- */

/* Sorted keep indices of every sequence (select_keep_indices,
 * tri/selection.py:108-196): protected prefix/recent windows are always kept;
 * policy GLOBAL keeps the top (budget - protected) scores of the middle;
 * policy V3 splits the middle into `segments` ranges with proportional
 * integer eviction quotas (tri/selection.py:165-189) and keeps each range's
 * top scores.  Ties at the selection threshold go to the lowest index.
 * scores: agg layout of kvc_aggregate.  keep: int64 [n_seq][keep_stride],
 * the first `budget` entries of each row written in ascending order.
 * The caller has validated budget/windows against every seq_len as the
 * reference does (tri/selection.py:123-133). */
int kvc_select_keep(kvc_stream_t stream, int n_seq, int max_seq_len, const int32_t* seq_lens,
                    const int64_t* token_offsets, const float* scores, int budget,
                    int protected_prefix, int protected_recent, int segments, int policy,
                    int64_t* keep, int64_t keep_stride);

/* The same selection with each (sequence, segment) cut into chunks of at least
 * 4096 scores, one workgroup per chunk (seven launches: reset, four radix
 * passes, per-chunk counts, emission), for batches of a few long sequences
 * that one workgroup per sequence would leave on a few CUs.  Identical output
 * to kvc_select_keep.  No counterpart in the reference beyond
 * select_keep_indices itself.  `workspace`: at least
 * kvc_select_workspace_bytes(n_seq, segments, policy) bytes, 16-byte aligned,
 * any contents (the first launch resets it); max_seq_len must bound every
 * sequence length. */
size_t kvc_select_workspace_bytes(int n_seq, int segments, int policy);
int kvc_select_keep_split(kvc_stream_t stream, int n_seq, int max_seq_len, const int32_t* seq_lens,
                          const int64_t* token_offsets, const float* scores, int budget,
                          int protected_prefix, int protected_recent, int segments, int policy,
                          int64_t* keep, int64_t keep_stride, void* workspace, size_t workspace_bytes);

/* ------------------------------------------------------------ compaction -- */

/* Move the kept K and V rows of every layer into their destinations
 * (token_slots + materialize_token_slots over all layers,
 * tri/method.py:272-288, tri/cache.py:9-15,100-112):
 *   row keep[b][i] of the source table  ->  row i of the destination table
 * for i < budget.  dst_block_ids == NULL selects in-place mode: destinations
 * are the front pages of the source table (dst page i/128 = source page i/128);
 * the kernel orders every read of a row before the write that overwrites it.
 * Otherwise destination pages must be private (disjoint from the source pages).
 * row_elems = kv_heads*head_dim; elem_bytes = 2.
 * workspace: NULL, or at least kvc_compact_workspace_bytes(n_seq, budget)
 * bytes, 16-byte aligned, any contents.  With it, batches of at most 32
 * sequences first resolve every kept row's source and destination offsets
 * into it and then move the rows one layer per workgroup (a small
 * address-translation working set: the same time whatever the physical
 * placement of the pool); in place, this covers the rows that follow the
 * ordered walk.  Without it, or for larger batches, a workgroup resolves its
 * rows once and walks every layer.  All forms give identical caches.
 * order: the dispatch order of the planned copy's per-layer workgroups,
 * KVC_COMPACT_LAYER_MAJOR (one layer after the other: few buffers in flight)
 * or KVC_COMPACT_LAYERS_INTERLEAVED (layer fastest, then row tile, sequence
 * slowest: every layer's buffers in flight at once).  Which is faster depends
 * on where the cache's pages sit in HBM (Qwen2.5-14B 16 x 16384 over fresh
 * allocations: layer-major 4.37-4.49 ms in all, interleaved 4.12-4.24 ms in
 * some and 4.59-4.77 ms in others), so a caller may time both on its cache.
 * The walked form ignores it. */
size_t kvc_compact_workspace_bytes(int n_seq, int budget);
int kvc_compact(kvc_stream_t stream, int n_layers, const uint64_t* k_layer_ptrs,
                const uint64_t* v_layer_ptrs, int64_t num_pages, int64_t page_stride,
                int64_t row_elems, int elem_bytes, int n_seq, const int32_t* seq_lens,
                const int64_t* src_block_offsets, const int64_t* src_block_ids,
                const int64_t* dst_block_offsets, const int64_t* dst_block_ids,
                const int64_t* keep, int64_t keep_stride, int budget, void* workspace,
                size_t workspace_bytes, int order);

/* New block table and released pages after compaction (PendingCompression and
 * the scheduler commit, pkg/provider.py:596-601, pkg/stateful.py:327-338):
 *   new_tables[b][j] = destination page j (j < ceil(budget/128))
 *   freed pages of b = reversed(source pages not reused), written at
 *   freed_ids[freed_offsets[b] ...]; in-place mode reuses the first
 *   ceil(budget/128) source pages, private mode releases every source page.
 * freed_offsets is computed by the caller (it knows the table lengths). */
int kvc_rewrite_block_tables(kvc_stream_t stream, int n_seq, int budget,
                             const int64_t* src_block_offsets, const int64_t* src_block_ids,
                             const int64_t* dst_block_offsets, const int64_t* dst_block_ids,
                             int64_t* new_tables, const int64_t* freed_offsets,
                             int64_t* freed_ids);

/* ------------------------------------------------------- slot utilities -- */

/* Logical token -> flat physical slot: block_ids[t/block_size]*block_size + t%block_size
 * (token_slots, tri/cache.py:9-15). Out-of-table tokens yield -1. */
int kvc_token_slots(kvc_stream_t stream, const int64_t* block_ids, int64_t n_blocks,
                    const int64_t* token_indices, int64_t n_tokens, int block_size,
                    int64_t* slots);

/* Scheduler page id -> consecutive 128-token kernel block ids:
 * out[i*k + j] = ids[i]*k + j (_expand_scheduler_block_ids, pkg/provider.py:1273-1287). */
int kvc_expand_block_ids(kvc_stream_t stream, const int64_t* ids, int64_t n_ids, int k,
                         int64_t* out);

/* Slot-addressed gather -> workspace -> scatter of K and V rows, safe for any
 * overlap between source and destination slots (materialize_token_slots,
 * tri/cache.py:100-112).  k_ws/v_ws hold n_slots*row_bytes bytes each. */
int kvc_materialize_slots(kvc_stream_t stream, void* k_cache, void* v_cache, int64_t num_pages,
                          int64_t page_stride, int64_t row_elems, int elem_bytes,
                          const int64_t* src_slots, const int64_t* dst_slots, int64_t n_slots,
                          void* k_ws, void* v_ws);

/* ------------------------------------------------- decode after compaction -- */

/* Physical positions of tokens written after a compaction (shift_positions,
 * tri/kernels.py:35-47; called by the slot-mapping hook pkg/provider.py:687-705):
 *   output[i] = positions[i] - request_offsets[request_indices[i]]
 * where request_offsets[r] = semantic length - physical length of request r
 * (pkg/provider.py:52-54).  request_indices are int32 (index_bytes 4) or int64
 * (index_bytes 8); positions, offsets and output are int64. */
int kvc_shift_positions(kvc_stream_t stream, const int64_t* positions, const void* request_indices,
                        int index_bytes, const int64_t* request_offsets, int64_t n, int64_t* output);

/* Slot mapping of one step's tokens from their physical positions: the
 * shift above fused with the host block table's compute_slot_mapping that the
 * reference hooks (pkg/plugin.py:487-506).  Request r owns tokens
 * [query_start_loc[r], query_start_loc[r+1]); with p = positions[i] -
 * request_offsets[r] (request_offsets may be NULL: no shift),
 *   slot_mapping[i] = block_table[r*block_table_stride + p/block_size]*block_size + p%block_size,
 * or -1 when p is negative, p/block_size >= max_blocks or the table entry is
 * negative.  Tokens in [query_start_loc[num_reqs], num_tokens) are padding and
 * get -1.  block_table is int32 (the host's layout); physical_positions, if
 * not NULL, receives p (positions[i] for padding). */
int kvc_physical_slot_mapping(kvc_stream_t stream, int num_reqs, const int32_t* query_start_loc,
                              const int64_t* positions, const int64_t* request_offsets,
                              const int32_t* block_table, int64_t block_table_stride, int max_blocks,
                              int block_size, int64_t num_tokens, int64_t* slot_mapping,
                              int64_t* physical_positions);

/* Physical attention lengths: seq_lens[r] -= request_offsets[r] for r < num_reqs,
 * in place, int32 (elem_bytes 4) or int64 (elem_bytes 8) lengths (device half of
 * apply_physical_attention_lengths, pkg/provider.py:707-728). */
int kvc_shift_lengths(kvc_stream_t stream, void* seq_lens, int elem_bytes, const int64_t* request_offsets,
                      int num_reqs);

/* ----------------------------------------------------------- calibration -- */

/* Query statistics of one layer's pre-RoPE query projections, accumulated over
 * tokens (_LayerAccumulator.add, pkg/calibration.py:98-131).  Element (t, h, d)
 * of q is at q[t*token_stride + h*head_dim + d] (dtype bf16, fp16 or fp32;
 * token_stride >= heads*head_dim, e.g. 2*heads*head_dim for a q_proj whose
 * output carries a gate after Q).  kvc_qstats_accumulate adds the tokens'
 * partial sums into `state` (kvc_qstats_state_bytes bytes, zeroed by the
 * caller before the first call); kvc_qstats_finish writes the totals over
 * every call so far.  With F = rotary_dim/2 and P = head_dim - rotary_dim, for
 * h < heads, f < F, p < P:
 *   real_sum[h*F + f] = sum_t q(t, h, f)
 *   imag_sum[h*F + f] = sum_t q(t, h, F + f)
 *   abs_sum[h*F + f]  = sum_t sqrt(q(t, h, f)^2 + q(t, h, F + f)^2)
 *   pass_sum[h*P + p] = sum_t q(t, h, rotary_dim + p)      (may be NULL if P == 0)
 * Each term is the reference's float32 value; the sums are float64 in an
 * order fixed by the shapes and the call sequence (identical on every run).
 * The caller keeps the token count. */
size_t kvc_qstats_state_bytes(int heads, int head_dim, int rotary_dim);
int kvc_qstats_accumulate(kvc_stream_t stream, int dtype, const void* q, int64_t n_tokens,
                          int64_t token_stride, int heads, int head_dim, int rotary_dim, void* state,
                          size_t state_bytes);
int kvc_qstats_finish(kvc_stream_t stream, int heads, int head_dim, int rotary_dim, const void* state,
                      double* real_sum, double* imag_sum, double* abs_sum, double* pass_sum);

#ifdef __cplusplus
}
#endif

#endif /* KVCOMPRESS_MI355X_H */
