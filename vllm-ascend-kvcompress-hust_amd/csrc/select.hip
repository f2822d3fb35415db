// Per-sequence keep-set selection on CDNA4: segmented radix select.
//
// Each workgroup owns one (sequence, segment).  The segment's scores are
// mapped to order-preserving 32-bit keys; four 8-bit radix passes build LDS
// histograms of the keys that still match the selected high digits and walk
// them from the top, which pins the exact key T of the K-th largest score and
// how many scores equal to T are still needed.  A last pass in index order
// keeps every key > T plus the first `need` keys == T (ties go to the lowest
// index), walking the segment in coalesced tiles: one workgroup prefix sum of
// packed (greater, equal) counts per tile gives every key its output slot, so
// the output is sorted without a sort.
//
// Segments follow select_keep_indices (tri/selection.py:108-196): the protected
// prefix [0, prefix) and recent window [n-recent, n) are always kept; policy
// GLOBAL keeps budget-prefix-recent of the middle; policy V3 cuts the middle
// into `segments` ranges [ms + M*k/S, ms + M*(k+1)/S) whose keep quota is
// len - (E*(stop-ms)/M - E*(start-ms)/M) with E = n - budget (integer floors).

#include "kvc_common.h"

namespace kvc {
namespace {

constexpr int kSelThreads = 1024;
constexpr int kSelWaves = kSelThreads / 64;
constexpr int kSelUnroll = 4;  // float4 words per thread in flight in a histogram pass
#ifndef KVC_SEL_PEEL
#define KVC_SEL_PEEL 1
#endif
constexpr int kSelPeel = KVC_SEL_PEEL;  // dominant digits counted with one atomic per wave
constexpr int kEmitWords = 2;  // float4 words per thread per emission tile
static_assert(kSelThreads * kEmitWords * 4 < 65536, "packed emission counts need 16 bits per half");

struct SelectArgs {
  int n_seq, budget, prefix, recent, segments, policy;
  const int32_t* seq_lens;
  const int64_t* token_offsets;
  const float* scores;
  int64_t* keep;
  int64_t keep_stride;
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

typedef float f32x4 __attribute__((ext_vector_type(4)));

// Calls f(i, key) for every i in [start, stop), spread over the workgroup:
// scalar head up to 16-byte alignment, float4 words kSelUnroll at a time
// (loads issued together), scalar tail.
template <typename F>
__device__ __forceinline__ void for_each_key(const float* sc, int64_t start, int64_t stop, F&& f) {
  const int tid = threadIdx.x;
  const int64_t misalign = (reinterpret_cast<uintptr_t>(sc + start) >> 2) & 3;
  int64_t head = (4 - misalign) & 3;
  if (head > stop - start) head = stop - start;
  for (int64_t i = start + tid; i < start + head; i += kSelThreads) f(i, float_key(sc[i]));
  const int64_t body = start + head;
  const int64_t n4 = (stop - body) >> 2;
  const f32x4* v = reinterpret_cast<const f32x4*>(sc + body);
  for (int64_t w0 = tid; w0 < n4; w0 += static_cast<int64_t>(kSelThreads) * kSelUnroll) {
    f32x4 x[kSelUnroll];
#pragma unroll
    for (int u = 0; u < kSelUnroll; ++u) {
      const int64_t w = w0 + static_cast<int64_t>(u) * kSelThreads;
      x[u] = v[w < n4 ? w : n4 - 1];  // in range; surplus words are ignored below
    }
#pragma unroll
    for (int u = 0; u < kSelUnroll; ++u) {
      const int64_t w = w0 + static_cast<int64_t>(u) * kSelThreads;
      if (w < n4) {
#pragma unroll
        for (int e = 0; e < 4; ++e) f(body + 4 * w + e, float_key(x[u][e]));
      }
    }
  }
  for (int64_t i = body + 4 * n4 + tid; i < stop; i += kSelThreads) f(i, float_key(sc[i]));
}

// Exclusive prefix sum over the workgroup (thread order); *total gets the sum.
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
  for (int w = 0; w < kSelWaves; ++w) {
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

__global__ __launch_bounds__(kSelThreads) void select_kernel(SelectArgs a) {
  __shared__ uint32_t whist[kSelWaves][256];
  __shared__ uint32_t hist[256];
  __shared__ uint32_t s_digit, s_need;
  __shared__ uint32_t s_wave[kSelWaves];

  const int b = blockIdx.y;
  const int seg = blockIdx.x;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int64_t n = a.seq_lens[b];
  const int64_t prefix = min(static_cast<int64_t>(a.prefix), n);
  const int64_t recent = min(static_cast<int64_t>(a.recent), n - prefix);
  const int64_t ms = prefix;
  const int64_t mc = n - prefix - recent;
  const int64_t evict = n - a.budget;
  const int nseg = (a.policy == KVC_POLICY_V3) ? a.segments : 1;
  if (seg >= nseg) return;
  int64_t* out = a.keep + static_cast<int64_t>(b) * a.keep_stride;
  const float* sc = a.scores + a.token_offsets[b];

  if (seg == 0) {
    for (int64_t i = tid; i < prefix; i += kSelThreads) out[i] = i;
    for (int64_t i = tid; i < recent; i += kSelThreads) out[a.budget - recent + i] = n - recent + i;
  }

  Segment s;
  int64_t out_base = prefix;
  if (a.policy == KVC_POLICY_V3) {
    if (mc <= 0) return;
    for (int k = 0; k < seg; ++k) out_base += v3_segment(ms, mc, evict, k, nseg).keep;
    s = v3_segment(ms, mc, evict, seg, nseg);
  } else {
    s.start = ms;
    s.stop = ms + mc;
    s.keep = a.budget - prefix - recent;
  }
  const int64_t len = s.stop - s.start;
  if (s.keep <= 0 || len <= 0) return;
  // Output rows are budget entries wide; the guards below keep a caller that
  // skipped validation (a sequence shorter than the budget) inside its row.
  if (s.keep >= len) {
    for (int64_t i = tid; i < len && out_base + i < a.budget; i += kSelThreads) out[out_base + i] = s.start + i;
    return;
  }

  // ---- radix select of the K-th largest key --------------------------------
  // Each wave counts into its own LDS histogram (keys of similar scores share
  // their high digits, so one shared histogram would serialise the atomics).
  uint32_t want = 0, mask = 0;
  uint32_t need = static_cast<uint32_t>(s.keep);
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = 24 - 8 * pass;
    for (int i = tid; i < kSelWaves * 256; i += kSelThreads) (&whist[0][0])[i] = 0;
    __syncthreads();
    uint32_t* mine = whist[wave];
    for_each_key(sc, s.start, s.stop, [&](int64_t, uint32_t k) {
      if ((k & mask) == want) count_digit(mine, (k >> shift) & 255u);
    });
    __syncthreads();
    if (tid < 256) {
      uint32_t c = 0;
#pragma unroll
      for (int w = 0; w < kSelWaves; ++w) c += whist[w][tid];
      hist[tid] = c;
    }
    __syncthreads();
    if (tid < 64) {
      // Lane l owns bins 4l..4l+3; `above` counts matching keys in higher bins.
      const uint32_t c0 = hist[4 * lane], c1 = hist[4 * lane + 1];
      const uint32_t c2 = hist[4 * lane + 2], c3 = hist[4 * lane + 3];
      const uint32_t tot = c0 + c1 + c2 + c3;
      uint32_t incl = tot;  // sum over lanes >= lane
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const uint32_t v = __shfl_down(incl, off);
        if (lane + off < 64) incl += v;
      }
      uint32_t above = incl - tot;
      const uint32_t cs[4] = {c0, c1, c2, c3};
#pragma unroll
      for (int j = 3; j >= 0; --j) {
        if (above < need && need <= above + cs[j]) {
          s_digit = static_cast<uint32_t>(4 * lane + j);
          s_need = need - above;
        }
        above += cs[j];
      }
    }
    __syncthreads();
    want |= s_digit << shift;
    mask |= 0xFFu << shift;
    need = s_need;
    __syncthreads();
  }
  const uint32_t thresh = want;   // exact key of the K-th largest score
  const uint32_t need_eq = need;  // keys equal to thresh that are kept

  // ---- ordered emission --------------------------------------------------
  // Key i is kept iff k > T, or k == T and fewer than need_eq ties precede it
  // (ties go to the lowest index); its output slot is G(i) + min(E(i), need_eq),
  // with G(i), E(i) the numbers of keys > T and == T before i in the segment.
  // The segment is walked in tiles of kSelThreads * kEmitWords float4 words:
  // thread t takes the tile's words [t*kEmitWords, (t+1)*kEmitWords), so the
  // loads are coalesced and thread order is index order, and one workgroup scan
  // of packed (G, E) counts per tile gives every thread its G and E.  The up to
  // three keys before the first 16-byte boundary and after the last are counted
  // by every thread and written by thread 0.
  uint32_t g_run = 0, e_run = 0;  // G and E at the current position (uniform)
  auto emit = [&](int64_t i, uint32_t k, uint32_t g, uint32_t e) {
    if (k > thresh || (k == thresh && e < need_eq)) {
      const int64_t slot = out_base + g + min(e, need_eq);
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
  const int64_t misalign = (reinterpret_cast<uintptr_t>(sc + s.start) >> 2) & 3;
  const int64_t head = min((4 - misalign) & 3, len);
  serial(s.start, s.start + head);
  const int64_t body = s.start + head;
  const int64_t n4 = (s.stop - body) >> 2;
  const f32x4* v = reinterpret_cast<const f32x4*>(sc + body);
  for (int64_t w0 = 0; w0 < n4; w0 += static_cast<int64_t>(kSelThreads) * kEmitWords) {
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
    // Per-tile counts stay below 2^16 (kSelThreads * kEmitWords * 4 keys), so
    // the two halves of the packed sum never carry into each other.
    const uint32_t before = block_exclusive_scan(g | (e << 16), s_wave, &tile_total);
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
  serial(body + 4 * n4, s.stop);
}

}  // namespace
}  // namespace kvc

using namespace kvc;

extern "C" int kvc_select_keep(kvc_stream_t stream, int n_seq, int max_seq_len,
                               const int32_t* seq_lens, const int64_t* token_offsets,
                               const float* scores, int budget, int protected_prefix,
                               int protected_recent, int segments, int policy, int64_t* keep,
                               int64_t keep_stride) {
  if (n_seq <= 0 || n_seq > 65535) return fail(KVC_EINVAL, "kvc_select_keep: bad n_seq %d", n_seq);
  if (budget <= 0 || budget > max_seq_len)
    return fail(KVC_EINVAL, "kvc_select_keep: budget must be in [1, max_seq_len]");
  if (protected_prefix < 0 || protected_recent < 0)
    return fail(KVC_EINVAL, "kvc_select_keep: protected windows must be non-negative");
  if (static_cast<int64_t>(protected_prefix) + protected_recent > budget)
    return fail(KVC_EINVAL, "kvc_select_keep: protected windows cannot exceed the budget");
  if (segments <= 0) return fail(KVC_EINVAL, "kvc_select_keep: segments must be positive");
  if (policy != KVC_POLICY_GLOBAL && policy != KVC_POLICY_V3)
    return fail(KVC_EINVAL, "kvc_select_keep: unknown policy %d", policy);
  if (keep_stride < budget) return fail(KVC_EINVAL, "kvc_select_keep: keep_stride < budget");
  if (!seq_lens || !token_offsets || !scores || !keep)
    return fail(KVC_EINVAL, "kvc_select_keep: null pointer");
  SelectArgs sa;
  sa.n_seq = n_seq;
  sa.budget = budget;
  sa.prefix = protected_prefix;
  sa.recent = protected_recent;
  sa.segments = segments;
  sa.policy = policy;
  sa.seq_lens = seq_lens;
  sa.token_offsets = token_offsets;
  sa.scores = scores;
  sa.keep = keep;
  sa.keep_stride = keep_stride;
  const int nseg = policy == KVC_POLICY_V3 ? segments : 1;
  dim3 grid(static_cast<unsigned>(nseg), static_cast<unsigned>(n_seq));
  select_kernel<<<grid, kSelThreads, 0, as_stream(stream)>>>(sa);
  return launch_status("kvc_select_keep");
}
