// Scorer definitions shared by the VALU (score.hip) and MFMA (score_mfma.hip) kernels.
#pragma once

#include "kvc_common.h"

namespace kvc {

constexpr int kScoreTile = 256;  // tokens per scoring workgroup
constexpr int kScoreThreads = 256;  // 4 waves
constexpr int kUnroll = 4;          // token iterations with loads in flight
static_assert(kScoreTile % kBlockSize == 0, "a scoring span starts and ends on page boundaries");
constexpr int kSpanPages = kScoreTile / kBlockSize;  // cache pages under one workgroup's span

// Base addresses of the pages under a workgroup's token span [t0, t0 + kScoreTile),
// resolved once before the token loop so that no K load waits on a block-table
// load (vector loads complete in issue order, so a table load issued inside the
// loop would also wait for every K load in flight before it).  A page that is
// past the table or out of the pool reads as zeros, as before.
struct SpanPages {
  KVC_GLOBAL const uint16_t* base[kSpanPages];
  bool ok[kSpanPages];

  __device__ __forceinline__ void resolve(KVC_GLOBAL const uint16_t* kbase, const int64_t* bt, int64_t n_blocks,
                                          int64_t num_pages, int64_t page_stride, int t0) {
#pragma unroll
    for (int i = 0; i < kSpanPages; ++i) {
      const int64_t blk = (t0 >> kBlockShift) + i;
      const int64_t p = blk < n_blocks ? bt[blk] : -1;
      ok[i] = p >= 0 && p < num_pages;
      base[i] = kbase + (ok[i] ? p : 0) * page_stride;
    }
  }
  // Page of span-relative token `rel` (0 <= rel < kScoreTile); unrolled selects, no indexing.
  __device__ __forceinline__ KVC_GLOBAL const uint16_t* page(int rel, bool* valid) const {
    const int idx = rel >> kBlockShift;
    KVC_GLOBAL const uint16_t* b = base[0];
    bool v = ok[0];
#pragma unroll
    for (int i = 1; i < kSpanPages; ++i) {
      if (idx == i) {
        b = base[i];
        v = ok[i];
      }
    }
    *valid = v;
    return b;
  }
};

struct ScoreShape {
  int n_layers, kv_heads, head_dim, rotary_dim, qpk;
  int freq, pass, units_rot, units, group_shift;
  int n_seq, max_tiles;
};

inline bool make_shape(ScoreShape* s, int n_layers, int kv_heads, int head_dim, int rotary_dim, int qpk,
                int n_seq, int max_seq_len) {
  if (n_layers <= 0 || kv_heads <= 0 || head_dim <= 0 || qpk <= 0 || qpk > 8 || n_seq <= 0 ||
      max_seq_len < 0)
    return false;
  if (rotary_dim <= 0 || rotary_dim > head_dim || rotary_dim % 16 != 0) return false;
  const int freq = rotary_dim / 2;
  const int pass = head_dim - rotary_dim;
  if (pass % 16 != 0) return false;
  s->n_layers = n_layers;
  s->kv_heads = kv_heads;
  s->head_dim = head_dim;
  s->rotary_dim = rotary_dim;
  s->qpk = qpk;
  s->freq = freq;
  s->pass = pass;
  s->units_rot = freq / 8;
  s->units = freq / 8 + pass / 16;
  int need = s->units > qpk ? s->units : qpk;
  int shift = 3;  // lane groups of 8, 16 or 32 lanes
  while ((1 << shift) < need) ++shift;
  if (shift > 5) return false;  // a head row must fit in 32 lanes
  s->group_shift = shift;
  // A workgroup covers every KV head of a token; groups beyond the last whole
  // token slot stay idle.
  const int groups_per_wg = (kScoreThreads / 64) * (64 >> shift);
  if (groups_per_wg < kv_heads) return false;
  s->n_seq = n_seq;
  s->max_tiles = static_cast<int>(ceil_div(max_seq_len, kScoreTile));
  return true;
}

inline size_t weights_floats(const ScoreShape& s) {
  return static_cast<size_t>(s.n_seq) * s.n_layers * s.kv_heads * s.units * 3 * s.qpk * 8;
}
// MFMA fragments: per (sequence, layer, KV head), 2*(head_dim/32) linear and
// 2*(F/32) |k| fragments (16-bit hi/lo), each holding the 16-byte words of the
// 4*qpk lanes of live query heads; then one float per (sequence, layer, KV
// head, query head): the column scale the fp16 fragments are divided by.
inline size_t mfma_fragment_only_bytes(const ScoreShape& s) {
  if (s.head_dim % 32 != 0 || s.freq % 32 != 0) return 0;
  const size_t frags = 2 * static_cast<size_t>(s.head_dim / 32) + 2 * static_cast<size_t>(s.freq / 32);
  return static_cast<size_t>(s.n_seq) * s.n_layers * s.kv_heads * frags * 4 * s.qpk * 16;
}
inline size_t mfma_fragment_bytes(const ScoreShape& s) {
  const size_t frag = mfma_fragment_only_bytes(s);
  if (frag == 0) return 0;
  return frag + static_cast<size_t>(s.n_seq) * s.n_layers * s.kv_heads * s.qpk * sizeof(float);
}
// The weight region holds either layout.
inline size_t weights_bytes_aligned(const ScoreShape& s) {
  const size_t valu = weights_floats(s) * sizeof(float);
  const size_t mfma = mfma_fragment_bytes(s);
  return ((valu > mfma ? valu : mfma) + 255) / 256 * 256;
}
inline size_t partial_count(const ScoreShape& s) {
  return static_cast<size_t>(s.n_layers) * s.n_seq * (s.max_tiles > 0 ? s.max_tiles : 1) *
         s.kv_heads * s.qpk;
}
inline size_t workspace_bytes(const ScoreShape& s) {
  return weights_bytes_aligned(s) + partial_count(s) * 2 * sizeof(double);
}
// Max-over-offsets scorer: after the mean scorer's workspace (whose weight
// region holds the magnitude and pass fragments and whose partial sums feed
// kvc_head_stats unchanged), the per-offset rotary fragments
// [n_seq][n_layers][kv_heads][qpk][chunk][step][hi/lo][64 lanes] of 16 bytes,
// chunk = 16 offsets and step = 32 rotary dims, then one float column scale
// per (sequence, layer, KV head, query head).
inline int offset_chunks(int n_offsets) { return (n_offsets + 15) / 16; }
inline size_t offset_fragment_bytes(const ScoreShape& s, int n_offsets) {
  return static_cast<size_t>(s.n_seq) * s.n_layers * s.kv_heads * s.qpk * offset_chunks(n_offsets) * (s.freq / 16) *
         2 * 64 * 16;
}
inline size_t max_tail_offset(const ScoreShape& s) { return (workspace_bytes(s) + 255) / 256 * 256; }
inline size_t max_workspace_bytes(const ScoreShape& s, int n_offsets) {
  const size_t frag = (offset_fragment_bytes(s, n_offsets) + 255) / 256 * 256;
  return max_tail_offset(s) + frag + static_cast<size_t>(s.n_seq) * s.n_layers * s.kv_heads * s.qpk * sizeof(float);
}


struct FoldArgs {
  int n_seq, n_layers, kv_heads, qpk, freq, pass, units_rot, units, rotary_dim, interleaved;
  int zero_rotary;  // 1: rotary linear weights are 0 (the max scorer adds its own rotary term)
  const float* q_real;
  const float* q_imag;
  const float* scale;
  const float* extra;
  const float* q_pass;
  const float* phase_cos;
  const float* phase_sin;
  int64_t phase_seq_stride;
  float* weights;  // [n_seq][n_layers][kv_heads][units][3][qpk][8]
};

struct ScoreArgs {
  const uint64_t* k_layer_ptrs;
  int64_t num_pages, page_stride;
  int kv_heads, head_dim, rotary_dim, freq;
  int units_rot, units, group_shift;
  int n_seq, max_tiles, n_layers;
  const int32_t* seq_lens;
  const int64_t* token_offsets;
  const int64_t* block_offsets;
  const int64_t* block_ids;
  const float* weights;
  float* raw;
  int64_t raw_layer_stride, raw_token_stride, raw_head_stride;
  double* partials;  // [n_layers][n_seq][max_tiles][kv_heads*QPK][2]
};

// MFMA scorer (score_mfma.hip): whether it serves this shape, and its launch
// (weight fold into bf16 or fp16 hi/lo fragments + scoring).  Returns a C-ABI code.
bool mfma_scorer_supported(const ScoreShape& s, int dtype, int rope_style);
int launch_mfma_scorer(hipStream_t stream, const ScoreShape& s, int dtype, const FoldArgs& fa, const ScoreArgs& sa,
                       void* weights);
// Max-over-offsets scorer (score_max.hip): fold of the per-offset fragments,
// magnitude/pass fold (zero_rotary) and scoring.  `fa.phase_cos/phase_sin`
// are the per-offset tables [n_seq][n_layers][n_offsets][F].
int launch_max_scorer(hipStream_t stream, const ScoreShape& s, int dtype, int n_offsets, const FoldArgs& fa,
                      const ScoreArgs& sa, void* workspace);
// The weight fold alone: bf16 or fp16 hi/lo fragments (and fp16 column scales)
// into `weights`, laid out as the MFMA scorer reads them.
int launch_mfma_fold(hipStream_t stream, const ScoreShape& s, int dtype, const FoldArgs& fa, void* weights);

// A dispatch's grid size in work-items is a 32-bit field of the dispatch
// packet; every launch of the scorers checks its own grid against it before
// the first launch of an entry point.
constexpr int64_t kMaxDispatchItems = 0xffffffffLL;
// Work-items of launch_mfma_fold's dispatch for this shape and dtype.
int64_t mfma_fold_items(const ScoreShape& s, int dtype);

}  // namespace kvc
