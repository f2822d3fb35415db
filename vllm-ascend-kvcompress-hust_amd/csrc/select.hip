// Per-sequence keep-set selection on CDNA4: segmented radix select.
//
// A job is one (sequence, segment).  The segment's scores are mapped to
// order-preserving 32-bit keys; four 8-bit radix passes build LDS histograms
// of the keys that still match the selected high digits and walk them from
// the top, which pins the exact key T of the K-th largest score and how many
// scores equal to T are still needed.  Emission keeps every key > T plus the
// first `need` keys == T (ties go to the lowest index), walking the segment in
// coalesced tiles: one workgroup prefix sum of packed (greater, equal) counts
// per tile gives every key its output slot, so the output is sorted without a
// sort.
//
// Two launch shapes:
//  * kvc_select_keep: one 1024-thread workgroup per job; every pass stays in
//    the workgroup.  Right for batches of many sequences.
//  * kvc_select_keep_split: a job's segment is cut into chunks of >= 4096 keys,
//    one 256-thread workgroup each.  Every radix pass is a launch: workgroups
//    add their chunk histograms into the pass's histogram in the workspace;
//    every workgroup of a later launch picks the earlier passes' digits
//    itself from those finished histograms (no workgroup waits for another).
//    Then one launch counts each chunk's keys > T and == T and one emits,
//    each chunk starting from the counts of the chunks before it.  Right for
//    a few long sequences, which would otherwise run on a few CUs.
// Both produce the same indices.
//
// Segments follow select_keep_indices (tri/selection.py:108-196): the protected
// prefix [0, prefix) and recent window [n-recent, n) are always kept; policy
// GLOBAL keeps budget-prefix-recent of the middle; policy V3 cuts the middle
// into `segments` ranges [ms + M*k/S, ms + M*(k+1)/S) whose keep quota is
// len - (E*(stop-ms)/M - E*(start-ms)/M) with E = n - budget (integer floors).

#include "kvc_common.h"

namespace kvc {
namespace {

constexpr int kSelThreads = 1024;   // one workgroup per job
constexpr int kSplitThreads = 256;  // split path: one workgroup per chunk
constexpr int kSplitChunk = 4096;   // keys per chunk, at least
constexpr int kSplitMaxChunks = 64;
constexpr int kSelUnroll = 4;  // float4 words per thread in flight in a histogram pass
constexpr int kEmitWords = 2;  // float4 words per thread per emission tile
constexpr int kSelPeel = 1;    // dominant digits counted with one atomic per wave
static_assert(kSelThreads * kEmitWords * 4 < 65536, "packed emission counts need 16 bits per half");

struct SelectArgs {
  int n_seq, budget, prefix, recent, segments, policy;
  const int32_t* seq_lens;
  const int64_t* token_offsets;
  const float* scores;
  int64_t* keep;
  int64_t keep_stride;
  void* state;  // split path: [n_seq][segments] SplitState
};

struct Segment {
  int64_t start, stop, keep;
};

__device__ Segment v3_segment(int64_t ms, int64_t mc, int64_t evict, int k, int nseg) {
  Segment s;
  s.start = ms + mc * k / nseg;
  s.stop = ms + mc * (k + 1) / nseg;
  const int64_t len = s.stop - s.start;
  if (len <= 0) {
    s.keep = 0;
    return s;
  }
  const int64_t before = evict * (s.start - ms) / mc;
  const int64_t after = evict * (s.stop - ms) / mc;
  const int64_t keep = len - (after - before);
  s.keep = keep > 0 ? keep : 0;
  return s;
}

// One (sequence, segment): its segment, first output slot and protected windows.
struct Job {
  int64_t n, prefix, recent, out_base;
  Segment s;
  bool exists;  // the segment index is in range for the policy
};

__device__ Job make_job(const SelectArgs& a, int b, int seg) {
  Job j;
  j.n = a.seq_lens[b];
  j.prefix = min(static_cast<int64_t>(a.prefix), j.n);
  j.recent = min(static_cast<int64_t>(a.recent), j.n - j.prefix);
  const int64_t ms = j.prefix;
  const int64_t mc = j.n - j.prefix - j.recent;
  const int nseg = (a.policy == KVC_POLICY_V3) ? a.segments : 1;
  j.exists = seg < nseg;
  j.out_base = j.prefix;
  j.s = Segment{ms, ms, 0};
  if (!j.exists) return j;
  if (a.policy == KVC_POLICY_V3) {
    if (mc <= 0) return j;
    const int64_t evict = j.n - a.budget;
    for (int k = 0; k < seg; ++k) j.out_base += v3_segment(ms, mc, evict, k, nseg).keep;
    j.s = v3_segment(ms, mc, evict, seg, nseg);
  } else {
    j.s = Segment{ms, ms + mc, a.budget - j.prefix - j.recent};
  }
  return j;
}

// Protected windows (the workgroup of segment 0) and segments kept whole.
// Returns whether the job still needs a radix select.  Output rows are budget
// entries wide; the guards keep a caller that skipped validation (a sequence
// shorter than the budget) inside its row.
__device__ bool fill_fixed(const SelectArgs& a, const Job& j, int seg, int64_t* out, int tid, int nthreads) {
  if (seg == 0) {
    for (int64_t i = tid; i < j.prefix; i += nthreads) out[i] = i;
    for (int64_t i = tid; i < j.recent; i += nthreads) out[a.budget - j.recent + i] = j.n - j.recent + i;
  }
  const int64_t len = j.s.stop - j.s.start;
  if (!j.exists || j.s.keep <= 0 || len <= 0) return false;
  if (j.s.keep >= len) {
    for (int64_t i = tid; i < len && j.out_base + i < a.budget; i += nthreads) out[j.out_base + i] = j.s.start + i;
    return false;
  }
  return true;
}

typedef float f32x4 __attribute__((ext_vector_type(4)));

// Calls f(i, key) for every i in [start, stop), spread over a workgroup of T
// threads: scalar head up to 16-byte alignment, float4 words kSelUnroll at a
// time (loads issued together), scalar tail.
template <int T, typename F>
__device__ __forceinline__ void for_each_key(const float* sc, int64_t start, int64_t stop, F&& f) {
  const int tid = threadIdx.x;
  const int64_t misalign = (reinterpret_cast<uintptr_t>(sc + start) >> 2) & 3;
  int64_t head = (4 - misalign) & 3;
  if (head > stop - start) head = stop - start;
  for (int64_t i = start + tid; i < start + head; i += T) f(i, float_key(sc[i]));
  const int64_t body = start + head;
  const int64_t n4 = (stop - body) >> 2;
  const f32x4* v = reinterpret_cast<const f32x4*>(sc + body);
  for (int64_t w0 = tid; w0 < n4; w0 += static_cast<int64_t>(T) * kSelUnroll) {
    f32x4 x[kSelUnroll];
#pragma unroll
    for (int u = 0; u < kSelUnroll; ++u) {
      const int64_t w = w0 + static_cast<int64_t>(u) * T;
      x[u] = v[w < n4 ? w : n4 - 1];  // in range; surplus words are ignored below
    }
#pragma unroll
    for (int u = 0; u < kSelUnroll; ++u) {
      const int64_t w = w0 + static_cast<int64_t>(u) * T;
      if (w < n4) {
#pragma unroll
        for (int e = 0; e < 4; ++e) f(body + 4 * w + e, float_key(x[u][e]));
      }
    }
  }
  for (int64_t i = body + 4 * n4 + tid; i < stop; i += T) f(i, float_key(sc[i]));
}

// Exclusive prefix sum over a workgroup of T threads (thread order); *total
// gets the sum.  s_wave holds T/64 entries.
template <int T>
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t v, uint32_t* s_wave, uint32_t* total) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  uint32_t incl = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t u = __shfl_up(incl, off);
    if (lane >= off) incl += u;
  }
  if (lane == 63) s_wave[wave] = incl;
  __syncthreads();
  uint32_t before = 0, all = 0;
#pragma unroll
  for (int w = 0; w < T / 64; ++w) {
    const uint32_t t = s_wave[w];
    if (w < wave) before += t;
    all += t;
  }
  __syncthreads();  // s_wave is reused by the next scan
  *total = all;
  return before + incl - v;
}

// Counts one key's digit into a wave's LDS histogram.  Scores of similar
// magnitude share their high digits (the first pass sees little more than the
// sign and exponent), so most lanes of a wave can hit one or two bins; up to
// kSelPeel times, the lanes holding the first active lane's digit add their
// number with a single atomic, and the lanes left count one by one.
__device__ __forceinline__ void count_digit(uint32_t* hist, uint32_t digit) {
#pragma unroll
  for (int p = 0; p < kSelPeel; ++p) {
    const uint32_t lead = __builtin_amdgcn_readfirstlane(digit);
    const uint64_t same = __ballot(digit == lead);
    if (digit == lead) {
      if (__lane_id() == static_cast<unsigned>(__ffsll(static_cast<unsigned long long>(same)) - 1))
        atomicAdd(&hist[lead], static_cast<uint32_t>(__popcll(same)));
      return;
    }
  }
  atomicAdd(&hist[digit], 1u);
}

// Histogram (digit at `shift`) of the keys in [start, stop) that match
// (want, mask): each wave counts into whist[wave], then hist = their sum.
// Every thread of the workgroup calls it; hist is complete on return.
template <int T>
__device__ void range_histogram(const float* sc, int64_t start, int64_t stop, uint32_t want, uint32_t mask, int shift,
                                uint32_t (*whist)[256], uint32_t* hist) {
  const int tid = threadIdx.x;
  for (int i = tid; i < (T / 64) * 256; i += T) (&whist[0][0])[i] = 0;
  __syncthreads();
  uint32_t* mine = whist[tid >> 6];
  for_each_key<T>(sc, start, stop, [&](int64_t, uint32_t k) {
    if ((k & mask) == want) count_digit(mine, (k >> shift) & 255u);
  });
  __syncthreads();
  for (int i = tid; i < 256; i += T) {
    uint32_t c = 0;
#pragma unroll
    for (int w = 0; w < T / 64; ++w) c += whist[w][i];
    hist[i] = c;
  }
  __syncthreads();
}

// Wave 0: the digit whose bin holds the need-th largest matching key, and how
// many keys of that bin are still needed.  Lane l owns bins 4l..4l+3.
__device__ __forceinline__ void pick_digit(const uint32_t* hist, uint32_t need, uint32_t* s_digit, uint32_t* s_need) {
  const int lane = threadIdx.x & 63;
  const uint32_t c0 = hist[4 * lane], c1 = hist[4 * lane + 1];
  const uint32_t c2 = hist[4 * lane + 2], c3 = hist[4 * lane + 3];
  const uint32_t tot = c0 + c1 + c2 + c3;
  uint32_t incl = tot;  // sum over lanes >= lane
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t v = __shfl_down(incl, off);
    if (lane + off < 64) incl += v;
  }
  uint32_t above = incl - tot;  // matching keys in higher bins
  const uint32_t cs[4] = {c0, c1, c2, c3};
#pragma unroll
  for (int j = 3; j >= 0; --j) {
    if (above < need && need <= above + cs[j]) {
      *s_digit = static_cast<uint32_t>(4 * lane + j);
      *s_need = need - above;
    }
    above += cs[j];
  }
}

// Ordered emission of [start, stop) by a workgroup of T threads, given the
// numbers g_run, e_run of keys > thresh and == thresh before `start` in the
// segment.  Key i is kept iff k > thresh, or k == thresh and fewer than
// need_eq ties precede it; its slot is out_base + G(i) + min(E(i), need_eq).
// Tiles of T*kEmitWords float4 words: thread t takes the tile's words
// [t*kEmitWords, (t+1)*kEmitWords), so loads are coalesced and thread order is
// index order; one scan of packed (G, E) counts per tile.  The up to three
// keys before the first 16-byte boundary and after the last are counted by
// every thread and written by thread 0.
template <int T>
__device__ void emit_range(const float* sc, int64_t start, int64_t stop, uint32_t thresh, uint32_t need_eq,
                           uint32_t g_run, uint32_t e_run, int64_t* out, int64_t out_base, int budget,
                           uint32_t* s_wave) {
  const int tid = threadIdx.x;
  auto emit = [&](int64_t i, uint32_t k, uint32_t g, uint32_t e) {
    if (k > thresh || (k == thresh && e < need_eq)) {
      const int64_t slot = out_base + g + min(e, need_eq);
      if (slot < budget) out[slot] = i;
    }
  };
  auto serial = [&](int64_t i0, int64_t i1) {
    for (int64_t i = i0; i < i1; ++i) {
      const uint32_t k = float_key(sc[i]);
      if (tid == 0) emit(i, k, g_run, e_run);
      g_run += k > thresh;
      e_run += k == thresh;
    }
  };
  const int64_t misalign = (reinterpret_cast<uintptr_t>(sc + start) >> 2) & 3;
  const int64_t head = min((4 - misalign) & 3, stop - start);
  serial(start, start + head);
  const int64_t body = start + head;
  const int64_t n4 = (stop - body) >> 2;
  const f32x4* v = reinterpret_cast<const f32x4*>(sc + body);
  for (int64_t w0 = 0; w0 < n4; w0 += static_cast<int64_t>(T) * kEmitWords) {
    uint32_t k[kEmitWords][4];
    bool valid[kEmitWords];
    uint32_t g = 0, e = 0;
#pragma unroll
    for (int u = 0; u < kEmitWords; ++u) {
      const int64_t w = w0 + static_cast<int64_t>(tid) * kEmitWords + u;
      valid[u] = w < n4;
      const f32x4 x = v[valid[u] ? w : n4 - 1];  // in range; surplus words are masked
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        k[u][q] = float_key(x[q]);
        g += valid[u] && k[u][q] > thresh;
        e += valid[u] && k[u][q] == thresh;
      }
    }
    uint32_t tile_total;
    // Per-tile counts stay below 2^16 (T * kEmitWords * 4 keys), so the two
    // halves of the packed sum never carry into each other.
    const uint32_t before = block_exclusive_scan<T>(g | (e << 16), s_wave, &tile_total);
    uint32_t gb = g_run + (before & 0xFFFFu), eb = e_run + (before >> 16);
#pragma unroll
    for (int u = 0; u < kEmitWords; ++u) {
      const int64_t i0 = body + 4 * (w0 + static_cast<int64_t>(tid) * kEmitWords + u);
      if (!valid[u]) continue;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        emit(i0 + q, k[u][q], gb, eb);
        gb += k[u][q] > thresh;
        eb += k[u][q] == thresh;
      }
    }
    g_run += tile_total & 0xFFFFu;
    e_run += tile_total >> 16;
  }
  serial(body + 4 * n4, stop);
}

// ------------------------------------------------- one workgroup per job --

// Segments whose aligned body has at most kCacheTiles emission tiles (16 384
// scores at 1024 threads) are read once: each thread keeps its words of every
// tile in registers, in the emission's layout, and the four radix passes and
// the emission walk those (the up to three scores before the first and after
// the last 16-byte boundary are read again each time, as in the uncached
// walk).
constexpr int kCacheTiles = 2;

__global__ __launch_bounds__(kSelThreads) void select_kernel(SelectArgs a) {
  __shared__ uint32_t whist[kSelThreads / 64][256];
  __shared__ uint32_t hist[256];
  __shared__ uint32_t s_digit, s_need;
  __shared__ uint32_t s_wave[kSelThreads / 64];

  const int b = blockIdx.y;
  const int seg = blockIdx.x;
  const int tid = threadIdx.x;
  const Job j = make_job(a, b, seg);
  int64_t* out = a.keep + static_cast<int64_t>(b) * a.keep_stride;
  if (!fill_fixed(a, j, seg, out, tid, kSelThreads)) return;
  const float* sc = a.scores + a.token_offsets[b];

  constexpr int64_t kTileWords = static_cast<int64_t>(kSelThreads) * kEmitWords;
  const int64_t start = j.s.start, stop = j.s.stop;
  const int64_t misalign = (reinterpret_cast<uintptr_t>(sc + start) >> 2) & 3;
  const int64_t head = min((4 - misalign) & 3, stop - start);
  const int64_t body = start + head;
  const int64_t n4 = (stop - body) >> 2;
  const int64_t tail0 = body + 4 * n4;
  const f32x4* v = reinterpret_cast<const f32x4*>(sc + body);
  const bool cached = n4 <= kCacheTiles * kTileWords;
  uint32_t ck[kCacheTiles][kEmitWords][4];
  bool cv[kCacheTiles][kEmitWords];
  if (cached) {
#pragma unroll
    for (int t = 0; t < kCacheTiles; ++t) {
#pragma unroll
      for (int u = 0; u < kEmitWords; ++u) {
        const int64_t w = t * kTileWords + static_cast<int64_t>(tid) * kEmitWords + u;
        cv[t][u] = w < n4;
        const f32x4 x = cv[t][u] ? v[w] : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int q = 0; q < 4; ++q) ck[t][u][q] = float_key(x[q]);
      }
    }
  }

  uint32_t want = 0, mask = 0;
  uint32_t need = static_cast<uint32_t>(j.s.keep);
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = 24 - 8 * pass;
    if (cached) {
      for (int i = tid; i < (kSelThreads / 64) * 256; i += kSelThreads) (&whist[0][0])[i] = 0;
      __syncthreads();
      uint32_t* mine = whist[tid >> 6];
      auto count = [&](uint32_t k) {
        if ((k & mask) == want) count_digit(mine, (k >> shift) & 255u);
      };
      for (int64_t i = start + tid; i < body; i += kSelThreads) count(float_key(sc[i]));
#pragma unroll
      for (int t = 0; t < kCacheTiles; ++t)
#pragma unroll
        for (int u = 0; u < kEmitWords; ++u)
          if (cv[t][u]) {
#pragma unroll
            for (int q = 0; q < 4; ++q) count(ck[t][u][q]);
          }
      for (int64_t i = tail0 + tid; i < stop; i += kSelThreads) count(float_key(sc[i]));
      __syncthreads();
      for (int i = tid; i < 256; i += kSelThreads) {
        uint32_t c = 0;
#pragma unroll
        for (int w = 0; w < kSelThreads / 64; ++w) c += whist[w][i];
        hist[i] = c;
      }
      __syncthreads();
    } else {
      range_histogram<kSelThreads>(sc, start, stop, want, mask, shift, whist, hist);
    }
    if (tid < 64) pick_digit(hist, need, &s_digit, &s_need);
    __syncthreads();
    want |= s_digit << shift;
    mask |= 0xFFu << shift;
    need = s_need;
    __syncthreads();
  }
  // want: the exact key of the K-th largest score; need: its ties to keep.
  if (!cached) {
    emit_range<kSelThreads>(sc, start, stop, want, need, 0u, 0u, out, j.out_base, a.budget, s_wave);
    return;
  }
  // The cached emission: emit_range's walk with the tiles' words from registers.
  const uint32_t thresh = want, need_eq = need;
  uint32_t g_run = 0, e_run = 0;
  auto emit = [&](int64_t i, uint32_t k, uint32_t g, uint32_t e) {
    if (k > thresh || (k == thresh && e < need_eq)) {
      const int64_t slot = j.out_base + g + min(e, need_eq);
      if (slot < a.budget) out[slot] = i;
    }
  };
  auto serial = [&](int64_t i0, int64_t i1) {
    for (int64_t i = i0; i < i1; ++i) {
      const uint32_t k = float_key(sc[i]);
      if (tid == 0) emit(i, k, g_run, e_run);
      g_run += k > thresh;
      e_run += k == thresh;
    }
  };
  serial(start, body);
#pragma unroll
  for (int t = 0; t < kCacheTiles; ++t) {
    if (t * kTileWords >= n4) break;  // the same for every thread
    uint32_t g = 0, e = 0;
#pragma unroll
    for (int u = 0; u < kEmitWords; ++u)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        g += cv[t][u] && ck[t][u][q] > thresh;
        e += cv[t][u] && ck[t][u][q] == thresh;
      }
    uint32_t tile_total;
    const uint32_t before = block_exclusive_scan<kSelThreads>(g | (e << 16), s_wave, &tile_total);
    uint32_t gb = g_run + (before & 0xFFFFu), eb = e_run + (before >> 16);
#pragma unroll
    for (int u = 0; u < kEmitWords; ++u) {
      if (!cv[t][u]) continue;
      const int64_t i0 = body + 4 * (t * kTileWords + static_cast<int64_t>(tid) * kEmitWords + u);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        emit(i0 + q, ck[t][u][q], gb, eb);
        gb += ck[t][u][q] > thresh;
        eb += ck[t][u][q] == thresh;
      }
    }
    g_run += tile_total & 0xFFFFu;
    e_run += tile_total >> 16;
  }
  serial(tail0, stop);
}

// ------------------------------------------------------ split over chunks --

// Per-job scratch of the split path (in the caller's workspace): the job's
// keep count and liveness (set by the reset launch), each radix pass's
// histogram (the chunks' atomic sums) and each chunk's counts of keys > T and
// == T.
struct SplitState {
  uint32_t need, live, pad[2];
  uint32_t hist[4][256];
  uint32_t counts[kSplitMaxChunks][2];
};

__host__ __device__ inline int64_t split_chunk_len(int64_t len) {
  int64_t cs = (len + kSplitMaxChunks - 1) / kSplitMaxChunks;
  if (cs < kSplitChunk) cs = kSplitChunk;
  return (cs + 3) & ~int64_t(3);
}

__host__ __device__ inline int split_chunks(int64_t len) {
  return len <= 0 ? 0 : static_cast<int>((len + split_chunk_len(len) - 1) / split_chunk_len(len));
}

__device__ __forceinline__ SplitState* split_state(const SelectArgs& a, int b, int seg) {
  return static_cast<SplitState*>(a.state) + static_cast<int64_t>(b) * a.segments + seg;
}

// grid (segments, n_seq): protected windows, whole segments, and the job's
// scratch reset (the workspace may hold the previous call's values).
__global__ __launch_bounds__(kSplitThreads) void select_split_init_kernel(SelectArgs a) {
  const int b = blockIdx.y, seg = blockIdx.x, tid = threadIdx.x;
  SplitState* st = split_state(a, b, seg);
  const Job j = make_job(a, b, seg);
  int64_t* out = a.keep + static_cast<int64_t>(b) * a.keep_stride;
  const bool live = fill_fixed(a, j, seg, out, tid, kSplitThreads);
  uint32_t* words = reinterpret_cast<uint32_t*>(st);
  for (int i = tid; i < static_cast<int>(sizeof(SplitState) / 4); i += kSplitThreads) words[i] = 0;
  __syncthreads();
  if (tid == 0) {
    st->live = live ? 1u : 0u;
    st->need = live ? static_cast<uint32_t>(j.s.keep) : 0u;
  }
}

// The radix prefix (want, mask) and the number of keys still needed inside
// it after `passes` passes: each pass's digit picked from that pass's
// histogram, complete since an earlier launch, exactly as the last pass of
// that histogram would have picked it.  The histograms are read together,
// then walked in LDS.  Every thread calls it; the results are in `out` (LDS)
// on return.
struct Threshold {
  uint32_t want, mask, need, digit;
};
__device__ void derive_threshold(const SplitState* st, int passes, uint32_t (*s_hist)[256], Threshold* out) {
  const int tid = threadIdx.x;
  for (int i = tid; i < passes * 256; i += kSplitThreads) (&s_hist[0][0])[i] = (&st->hist[0][0])[i];
  if (tid == 0) *out = Threshold{0u, 0u, st->need, 0u};
  __syncthreads();
  for (int q = 0; q < passes; ++q) {
    if (tid < 64) {
      const uint32_t need = out->need;  // read by every lane before one lane writes
      pick_digit(s_hist[q], need, &out->digit, &out->need);
    }
    __syncthreads();
    if (tid == 0) {
      const int shift = 24 - 8 * q;
      out->want |= out->digit << shift;
      out->mask |= 0xFFu << shift;
    }
    __syncthreads();
  }
}

// grid (chunks, segments, n_seq): one radix pass.  Each workgroup derives the
// prefix of the passes before (from their histograms) and adds its chunk's
// histogram of the matching keys into the job's; no workgroup waits for
// another inside the launch.
__global__ __launch_bounds__(kSplitThreads) void select_split_pass_kernel(SelectArgs a, int pass) {
  __shared__ uint32_t whist[kSplitThreads / 64][256];
  __shared__ uint32_t hist[256];
  __shared__ uint32_t s_prev[3][256];
  __shared__ Threshold s_th;
  const int c = blockIdx.x, seg = blockIdx.y, b = blockIdx.z, tid = threadIdx.x;
  SplitState* st = split_state(a, b, seg);
  if (!st->live) return;  // the whole workgroup reads the same word
  const Job j = make_job(a, b, seg);
  const int64_t len = j.s.stop - j.s.start;
  const int chunks = split_chunks(len);
  if (c >= chunks) return;
  const int64_t cs = split_chunk_len(len);
  const int64_t c0 = j.s.start + c * cs, c1 = min(j.s.stop, c0 + cs);
  derive_threshold(st, pass, s_prev, &s_th);
  const int shift = 24 - 8 * pass;
  const float* sc = a.scores + a.token_offsets[b];
  range_histogram<kSplitThreads>(sc, c0, c1, s_th.want, s_th.mask, shift, whist, hist);
  for (int i = tid; i < 256; i += kSplitThreads)
    if (hist[i]) atomicAdd(&st->hist[pass][i], hist[i]);
}

// grid (chunks, segments, n_seq): each chunk's keys > T and == T.
__global__ __launch_bounds__(kSplitThreads) void select_split_count_kernel(SelectArgs a) {
  __shared__ uint32_t s_wave[kSplitThreads / 64];
  __shared__ uint32_t s_prev[4][256];
  __shared__ Threshold s_th;
  const int c = blockIdx.x, seg = blockIdx.y, b = blockIdx.z;
  SplitState* st = split_state(a, b, seg);
  if (!st->live) return;
  const Job j = make_job(a, b, seg);
  const int64_t len = j.s.stop - j.s.start;
  if (c >= split_chunks(len)) return;
  const int64_t cs = split_chunk_len(len);
  const int64_t c0 = j.s.start + c * cs, c1 = min(j.s.stop, c0 + cs);
  derive_threshold(st, 4, s_prev, &s_th);
  const uint32_t thresh = s_th.want;
  const float* sc = a.scores + a.token_offsets[b];
  uint32_t g = 0, e = 0;
  for_each_key<kSplitThreads>(sc, c0, c1, [&](int64_t, uint32_t k) {
    g += k > thresh;
    e += k == thresh;
  });
  uint32_t total_g, total_e;
  block_exclusive_scan<kSplitThreads>(g, s_wave, &total_g);
  block_exclusive_scan<kSplitThreads>(e, s_wave, &total_e);
  if (threadIdx.x == 0) {
    st->counts[c][0] = total_g;
    st->counts[c][1] = total_e;
  }
}

// grid (chunks, segments, n_seq): ordered emission of each chunk.
__global__ __launch_bounds__(kSplitThreads) void select_split_emit_kernel(SelectArgs a) {
  __shared__ uint32_t s_wave[kSplitThreads / 64];
  __shared__ uint32_t s_prev[4][256];
  __shared__ Threshold s_th;
  const int c = blockIdx.x, seg = blockIdx.y, b = blockIdx.z;
  SplitState* st = split_state(a, b, seg);
  if (!st->live) return;
  const Job j = make_job(a, b, seg);
  const int64_t len = j.s.stop - j.s.start;
  if (c >= split_chunks(len)) return;
  const int64_t cs = split_chunk_len(len);
  const int64_t c0 = j.s.start + c * cs, c1 = min(j.s.stop, c0 + cs);
  uint32_t g0 = 0, e0 = 0;
  for (int i = 0; i < c; ++i) {
    g0 += st->counts[i][0];
    e0 += st->counts[i][1];
  }
  derive_threshold(st, 4, s_prev, &s_th);
  int64_t* out = a.keep + static_cast<int64_t>(b) * a.keep_stride;
  emit_range<kSplitThreads>(a.scores + a.token_offsets[b], c0, c1, s_th.want, s_th.need, g0, e0, out, j.out_base,
                            a.budget, s_wave);
}

int check_select_args(const char* who, int n_seq, int max_seq_len, const int32_t* seq_lens,
                      const int64_t* token_offsets, const float* scores, int budget, int protected_prefix,
                      int protected_recent, int segments, int policy, int64_t* keep, int64_t keep_stride) {
  if (n_seq <= 0 || n_seq > 65535) return fail(KVC_EINVAL, "%s: bad n_seq %d", who, n_seq);
  if (budget <= 0 || budget > max_seq_len) return fail(KVC_EINVAL, "%s: budget must be in [1, max_seq_len]", who);
  if (protected_prefix < 0 || protected_recent < 0)
    return fail(KVC_EINVAL, "%s: protected windows must be non-negative", who);
  if (static_cast<int64_t>(protected_prefix) + protected_recent > budget)
    return fail(KVC_EINVAL, "%s: protected windows cannot exceed the budget", who);
  if (segments <= 0) return fail(KVC_EINVAL, "%s: segments must be positive", who);
  if (policy != KVC_POLICY_GLOBAL && policy != KVC_POLICY_V3)
    return fail(KVC_EINVAL, "%s: unknown policy %d", who, policy);
  if (keep_stride < budget) return fail(KVC_EINVAL, "%s: keep_stride < budget", who);
  if (!seq_lens || !token_offsets || !scores || !keep) return fail(KVC_EINVAL, "%s: null pointer", who);
  return 0;
}

SelectArgs make_select_args(int n_seq, const int32_t* seq_lens, const int64_t* token_offsets, const float* scores,
                            int budget, int protected_prefix, int protected_recent, int segments, int policy,
                            int64_t* keep, int64_t keep_stride) {
  SelectArgs sa;
  sa.n_seq = n_seq;
  sa.budget = budget;
  sa.prefix = protected_prefix;
  sa.recent = protected_recent;
  sa.segments = policy == KVC_POLICY_V3 ? segments : 1;
  sa.policy = policy;
  sa.seq_lens = seq_lens;
  sa.token_offsets = token_offsets;
  sa.scores = scores;
  sa.keep = keep;
  sa.keep_stride = keep_stride;
  sa.state = nullptr;
  return sa;
}

}  // namespace
}  // namespace kvc

using namespace kvc;

extern "C" int kvc_select_keep(kvc_stream_t stream, int n_seq, int max_seq_len,
                               const int32_t* seq_lens, const int64_t* token_offsets,
                               const float* scores, int budget, int protected_prefix,
                               int protected_recent, int segments, int policy, int64_t* keep,
                               int64_t keep_stride) {
  if (int rc = check_select_args("kvc_select_keep", n_seq, max_seq_len, seq_lens, token_offsets, scores, budget,
                                 protected_prefix, protected_recent, segments, policy, keep, keep_stride))
    return rc;
  const SelectArgs sa = make_select_args(n_seq, seq_lens, token_offsets, scores, budget, protected_prefix,
                                         protected_recent, segments, policy, keep, keep_stride);
  dim3 grid(static_cast<unsigned>(sa.segments), static_cast<unsigned>(n_seq));
  select_kernel<<<grid, kSelThreads, 0, as_stream(stream)>>>(sa);
  return launch_status("kvc_select_keep");
}

extern "C" size_t kvc_select_workspace_bytes(int n_seq, int segments, int policy) {
  if (n_seq <= 0 || segments <= 0) return 0;
  const int nseg = policy == KVC_POLICY_V3 ? segments : 1;
  return static_cast<size_t>(n_seq) * nseg * sizeof(SplitState);
}

extern "C" int kvc_select_keep_split(kvc_stream_t stream, int n_seq, int max_seq_len,
                                     const int32_t* seq_lens, const int64_t* token_offsets,
                                     const float* scores, int budget, int protected_prefix,
                                     int protected_recent, int segments, int policy, int64_t* keep,
                                     int64_t keep_stride, void* workspace, size_t workspace_bytes) {
  if (int rc = check_select_args("kvc_select_keep_split", n_seq, max_seq_len, seq_lens, token_offsets, scores,
                                 budget, protected_prefix, protected_recent, segments, policy, keep, keep_stride))
    return rc;
  const size_t need = kvc_select_workspace_bytes(n_seq, segments, policy);
  if (!workspace || workspace_bytes < need || reinterpret_cast<uintptr_t>(workspace) % 16)
    return fail(KVC_EINVAL, "kvc_select_keep_split: a 16-byte aligned workspace of %zu bytes is needed", need);
  SelectArgs sa = make_select_args(n_seq, seq_lens, token_offsets, scores, budget, protected_prefix,
                                   protected_recent, segments, policy, keep, keep_stride);
  sa.state = workspace;
  // A segment is at most the whole sequence.
  const int chunks = split_chunks(max_seq_len);
  hipStream_t st = as_stream(stream);
  select_split_init_kernel<<<dim3(sa.segments, n_seq), kSplitThreads, 0, st>>>(sa);
  if (int rc = launch_status("kvc_select_keep_split(init)")) return rc;
  const dim3 grid(static_cast<unsigned>(chunks), static_cast<unsigned>(sa.segments), static_cast<unsigned>(n_seq));
  for (int pass = 0; pass < 4; ++pass) {
    select_split_pass_kernel<<<grid, kSplitThreads, 0, st>>>(sa, pass);
    if (int rc = launch_status("kvc_select_keep_split(pass)")) return rc;
  }
  select_split_count_kernel<<<grid, kSplitThreads, 0, st>>>(sa);
  if (int rc = launch_status("kvc_select_keep_split(count)")) return rc;
  select_split_emit_kernel<<<grid, kSplitThreads, 0, st>>>(sa);
  return launch_status("kvc_select_keep_split(emit)");
}
