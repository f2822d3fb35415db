// Per-sequence keep-set selection on CDNA4: segmented radix select.
//
// Each workgroup owns one (sequence, segment).  The segment's scores are
// mapped to order-preserving 32-bit keys; four 8-bit radix passes build LDS
// histograms of the keys that still match the selected high digits and walk
// them from the top, which pins the exact key T of the K-th largest score and
// how many scores equal to T are still needed.  A last pass in index order
// keeps every key > T plus the first `need` keys == T (ties go to the lowest
// index) and writes the kept indices with wave ballots and a workgroup prefix
// sum, so the output is sorted without a sort.
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

__device__ __forceinline__ uint32_t lane_prefix(uint64_t mask, int lane) {
  return static_cast<uint32_t>(__popcll(mask & ((1ull << lane) - 1ull)));
}

__global__ __launch_bounds__(kSelThreads) void select_kernel(SelectArgs a) {
  __shared__ uint32_t hist[256];
  __shared__ uint32_t s_digit, s_need;
  __shared__ uint32_t w_take[kSelWaves], w_eq[kSelWaves];

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
  uint32_t want = 0, mask = 0;
  uint32_t need = static_cast<uint32_t>(s.keep);
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = 24 - 8 * pass;
    if (tid < 256) hist[tid] = 0;
    __syncthreads();
    for (int64_t i = s.start + tid; i < s.stop; i += kSelThreads) {
      const uint32_t k = float_key(sc[i]);
      if ((k & mask) == want) atomicAdd(&hist[(k >> shift) & 255u], 1u);
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
  const uint32_t thresh = want;  // exact key of the K-th largest score
  const uint32_t need_eq = need;  // keys equal to thresh that are kept

  // ---- ordered emission --------------------------------------------------
  uint32_t base_take = 0, base_eq = 0;
  for (int64_t chunk = s.start; chunk < s.stop; chunk += kSelThreads) {
    const int64_t i = chunk + tid;
    const bool in = i < s.stop;
    const uint32_t k = in ? float_key(sc[i]) : 0u;
    const bool gt = in && k > thresh;
    const bool eq = in && k == thresh;
    const uint64_t m_eq = __ballot(eq);
    if (lane == 0) w_eq[wave] = static_cast<uint32_t>(__popcll(m_eq));
    __syncthreads();
    uint32_t eq_before = base_eq + lane_prefix(m_eq, lane);
    uint32_t eq_total = 0;
    for (int w = 0; w < kSelWaves; ++w) {
      if (w < wave) eq_before += w_eq[w];
      eq_total += w_eq[w];
    }
    const bool take = gt || (eq && eq_before < need_eq);
    const uint64_t m_take = __ballot(take);
    if (lane == 0) w_take[wave] = static_cast<uint32_t>(__popcll(m_take));
    __syncthreads();
    uint32_t pos = base_take + lane_prefix(m_take, lane);
    uint32_t take_total = 0;
    for (int w = 0; w < kSelWaves; ++w) {
      if (w < wave) pos += w_take[w];
      take_total += w_take[w];
    }
    if (take && out_base + pos < a.budget) out[out_base + pos] = i;
    base_take += take_total;
    base_eq += eq_total;
    __syncthreads();
  }
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
