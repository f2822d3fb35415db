// TriAttention scores with score_aggregation = "max" on the matrix cores
// (tri/scoring.py:84-97): the rotary term is maximised over the future
// offsets instead of averaged,
//   score = max_o sum_f a[(qr kr + qi ki) cos(phi_of) - (qi kr - qr ki) sin(phi_of)]
//         + sum_f a*extra*|k_f| + q_pass.k_pass,      phi_of = (o + rs) * omega_f.
// For one offset the rotary term is a dot product of the key with per-offset
// folded weights, kr*a(qr c - qi s) + ki*a(qi c + qr s), so every (query
// head, offset) pair is one more column of the scoring GEMM.  Per query head
// the offsets fill chunks of 16 B columns (columns past the last offset repeat
// it, which leaves the maximum unchanged); a 16-token key tile times a chunk
// gives D[token][offset] with the 16 offsets of a row in the 16 lanes of a DPP
// row, so the maximum over offsets is an elementwise max across chunks and
// four DPP steps inside the row.  The magnitude and pass terms do not depend
// on the offset: they come from the mean scorer's fragments with the rotary
// weights set to zero and are added after the maximum, as in the reference.
//
// Work split: a workgroup owns one KV head, a group of its query heads (all of
// them when their fragments fit the LDS budget) and KVC_MAX_SPANS consecutive
// 256-token spans; its four waves walk interleaved 16-token tiles of a span.
// The per-offset fragments (bf16 or fp16 hi/lo, 1 KB per 32 rotary dims and
// chunk) are staged in LDS once per workgroup; each fragment read feeds two
// key tiles.  Workgroups that share a key span but not a query-head group are
// placed eight apart in the grid, on the same XCD, so the second read of the
// keys is an L2 hit.  Raw scores, partial sums and the stage epilogue are the
// mean scorer's.

#include <math.h>

#include "mfma_common.h"

#ifndef KVC_MAX_FRAG_LDS
#define KVC_MAX_FRAG_LDS (48 * 1024)  // bytes of per-offset fragments staged per workgroup
#endif
#ifndef KVC_MAX_SPANS
#define KVC_MAX_SPANS 4  // 256-token spans per workgroup
#endif

namespace kvc {
namespace {

constexpr int kMaxSpans = KVC_MAX_SPANS;
constexpr int kMaxFragLds = KVC_MAX_FRAG_LDS;
constexpr int kOffsetFragBytes = 64 * 16;  // one B operand: 64 lanes x 8 16-bit values

struct OffsetFoldArgs {
  FoldArgs f;  // calibration and shape; f.phase_cos/phase_sin are [b][l][o][F]
  int n_offsets, nch, nr;
  u32x4* frags;      // [col][chunk][step][hi/lo][64 lanes]
  float* inv_scale;  // [col]: 2^-s for fp16 columns scaled by 2^s, else 1
};

// Folded weight of rotary dim d (0 <= d < 2F) for offset o and calibration
// row `row` = (layer * kv_heads + head) * qpk + g.
__device__ __forceinline__ float offset_weight(const FoldArgs& a, int b, int layer, int64_t row, int o, int n_offsets,
                                               int d) {
  const bool real = a.interleaved ? (d & 1) == 0 : d < a.freq;
  const int f = a.interleaved ? d >> 1 : (d < a.freq ? d : d - a.freq);
  const int64_t ph = b * a.phase_seq_stride + (static_cast<int64_t>(layer) * n_offsets + o) * a.freq + f;
  const int64_t q = row * a.freq + f;
  const float qr = a.q_real[q], qi = a.q_imag[q], sc = a.scale[q];
  const float c = a.phase_cos[ph], sn = a.phase_sin[ph];
  return real ? sc * (qr * c - qi * sn) : sc * (qi * c + qr * sn);
}

// One wave per column (sequence, layer, KV head, query head g).  Lane l owns
// B-operand lane l of every (chunk, step) fragment: offset column 16*chunk +
// l%16 (clamped to the last offset), rotary dims 32*step + 8*(l/16) + e.  fp16
// columns are scaled by the power of two that brings their largest weight to
// [2^13, 2^14), as the mean scorer's fp16 fold does.
template <bool F16>
__global__ __launch_bounds__(256) void fold_offsets_kernel(OffsetFoldArgs m) {
  typedef MfmaElem<F16> E;
  const FoldArgs& a = m.f;
  const int64_t col = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int64_t cols = static_cast<int64_t>(a.n_seq) * a.n_layers * a.kv_heads * a.qpk;
  if (col >= cols) return;  // whole wave
  const int lane = threadIdx.x & 63;
  const int g = static_cast<int>(col % a.qpk);
  int64_t r = col / a.qpk;
  const int head = static_cast<int>(r % a.kv_heads);
  r /= a.kv_heads;
  const int layer = static_cast<int>(r % a.n_layers);
  const int b = static_cast<int>(r / a.n_layers);
  const int64_t row = (static_cast<int64_t>(layer) * a.kv_heads + head) * a.qpk + g;
  const int j = lane & 15, kb = lane >> 4;
  const int n_pos = m.nch * m.nr;
  int sh = 0;
  if (F16) {
    float big = 0.0f;
    for (int p = 0; p < n_pos; ++p) {
      const int c = p / m.nr, st = p - c * m.nr;
      const int o = min(16 * c + j, m.n_offsets - 1);
      for (int e = 0; e < 8; ++e)
        big = fmaxf(big, fabsf(offset_weight(a, b, layer, row, o, m.n_offsets, 32 * st + 8 * kb + e)));
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) big = fmaxf(big, __shfl_xor(big, off));
    if (big > 0.0f && big <= 3.4e38f) {
      int ex;
      (void)frexpf(big, &ex);  // big < 2^ex
      sh = 14 - ex;
      sh = sh < -126 ? -126 : (sh > 126 ? 126 : sh);
    }
  }
  u32x4* dst = m.frags + col * n_pos * 2 * 64 + lane;
  for (int p = 0; p < n_pos; ++p) {
    const int c = p / m.nr, st = p - c * m.nr;
    const int o = min(16 * c + j, m.n_offsets - 1);
    u32x4 hi, lo;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      float v0 = offset_weight(a, b, layer, row, o, m.n_offsets, 32 * st + 8 * kb + 2 * w);
      float v1 = offset_weight(a, b, layer, row, o, m.n_offsets, 32 * st + 8 * kb + 2 * w + 1);
      if (F16) {
        v0 = ldexpf(v0, sh);
        v1 = ldexpf(v1, sh);
      }
      const uint32_t h = E::pack(v0, v1);
      hi[w] = h;
      lo[w] = E::pack(v0 - E::lo(h), v1 - E::hi(h));
    }
    dst[(2 * p) * 64] = hi;
    dst[(2 * p + 1) * 64] = lo;
  }
  if (lane == 0) m.inv_scale[col] = F16 ? ldexpf(1.0f, -sh) : 1.0f;
}

struct MaxGeometry {
  int gpg;     // query heads per workgroup
  int groups;  // query-head groups per KV head
  int nch;     // 16-offset chunks
  int work;    // (span set, KV head) items
};

// Maximum over the 16 lanes of a DPP row (NaN-propagating, as torch.maximum).
__device__ __forceinline__ float row16_max(float v) {
  v = max_nan(v, dpp_quad_xor1(v));
  v = max_nan(v, dpp_quad_xor2(v));
  v = max_nan(v, dpp_row_half_mirror(v));
  v = max_nan(v, dpp_row_mirror(v));
  return v;
}

template <int NK, int NF, bool F16, bool IL>
__global__ __launch_bounds__(kScoreThreads) void score_max_kernel(ScoreArgs a, MaxGeometry geo, int qpk,
                                                                  const u32x4* __restrict__ rest_frags,
                                                                  const float* __restrict__ rest_scale,
                                                                  const u32x4* __restrict__ off_frags,
                                                                  const float* __restrict__ off_scale) {
  typedef MfmaElem<F16> E;
  typedef typename E::vec vec_t;
  constexpr int NR = 2 * NF;                    // rotary K steps of 32 dims
  constexpr int NP = NK - NR;                   // pass K steps
  constexpr int kNP = NP > 0 ? NP : 1;
  extern __shared__ u32x4 lds_frag[];           // [gpg][nch][NR][hi/lo][64]

  // blockIdx.x = ((item / 8) * groups + group) * 8 + item % 8: the groups of
  // one item are eight workgroups apart (same XCD).
  const int p = blockIdx.x;
  const int gg = (p >> 3) % geo.groups;
  const int item = ((p >> 3) / geo.groups) * 8 + (p & 7);
  if (item >= geo.work) return;
  const int head = item % a.kv_heads;
  const int tile_first = (item / a.kv_heads) * kMaxSpans;
  const int layer = blockIdx.z;
  const int b = blockIdx.y;
  const int n = a.seq_lens[b];
  if (tile_first * kScoreTile >= n) return;  // whole workgroup leaves together
  const int g0 = gg * geo.gpg;
  const int gcnt = min(geo.gpg, qpk - g0);
  if (gcnt <= 0) return;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r = lane & 15;   // A row (token in tile) / D column
  const int kb = lane >> 4;  // K block of A/B, row block of D
  const int64_t col0 = ((static_cast<int64_t>(b) * a.n_layers + layer) * a.kv_heads + head) * qpk;
  const int frag_per_g = geo.nch * NR * 2 * 64;

  // Stage this group's per-offset fragments.
  {
    const u32x4* src = off_frags + (col0 + g0) * frag_per_g;
    const int count = gcnt * frag_per_g;
#pragma unroll 4
    for (int i = threadIdx.x; i < count; i += kScoreThreads) lds_frag[i] = src[i];
  }

  // Magnitude and pass fragments (packed [frag][kb][g < qpk], rotary weights zero).
  constexpr int kFrags = 2 * NK + 2 * NF;
  const int packed = 4 * qpk;
  const bool live_col = r < qpk;
  const u32x4* fp = rest_frags + (((static_cast<int64_t>(b) * a.n_layers + layer) * a.kv_heads + head) * kFrags) * packed +
                    kb * qpk + (live_col ? r : 0);
  auto frag_word = [&](int f) {
    const u32x4 v = fp[f * packed];
    return __builtin_bit_cast(vec_t, live_col ? v : u32x4{0, 0, 0, 0});
  };
  vec_t p_hi[kNP], p_lo[kNP], m_hi[NF], m_lo[NF];
#pragma unroll
  for (int j = 0; j < NP; ++j) {
    p_hi[j] = frag_word(2 * (NR + j));
    p_lo[j] = frag_word(2 * (NR + j) + 1);
  }
#pragma unroll
  for (int q = 0; q < NF; ++q) {
    m_hi[q] = frag_word(2 * NK + 2 * q);
    m_lo[q] = frag_word(2 * NK + 2 * q + 1);
  }
  const float r_scale = F16 ? rest_scale[col0 + (live_col ? r : 0)] : 1.0f;
  const float o_scale = F16 ? off_scale[col0 + (live_col ? r : 0)] : 1.0f;

  KVC_GLOBAL const uint16_t* kbase = gptr_from_int<const uint16_t>(a.k_layer_ptrs[layer]);
  const int64_t* bt = a.block_ids + a.block_offsets[b];
  const int64_t n_blocks = a.block_offsets[b + 1] - a.block_offsets[b];
  const int64_t row_elems = static_cast<int64_t>(a.kv_heads) * a.head_dim;
  const int64_t lane_off = static_cast<int64_t>(head) * a.head_dim + 8 * kb;
  const int64_t tok_base = a.token_offsets[b];
  float* raw_out = a.raw + layer * a.raw_layer_stride;
  const bool writer = r >= g0 && r < g0 + gcnt;

  __shared__ __attribute__((aligned(16))) float stage[kMfmaMaxQpk * kStageStride];
  __shared__ double red[2][kScoreThreads];
  float* stage_row = stage + (writer ? r - g0 : 0) * kStageStride;
  __syncthreads();  // fragments staged

  // Magnitude + pass term of a tile: D[4*kb + i][r] for query head r.
  auto rest_tile = [&](const u32x4 (&ka)[NK]) {
    f32x4 acc0 = {0.0f, 0.0f, 0.0f, 0.0f};
    f32x4 acc1 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < NP; ++j) {
      const vec_t kv = __builtin_bit_cast(vec_t, ka[NR + j]);
      if (j & 1) {
        acc1 = E::mfma(kv, p_hi[j], acc1);
        acc1 = E::mfma(kv, p_lo[j], acc1);
      } else {
        acc0 = E::mfma(kv, p_hi[j], acc0);
        acc0 = E::mfma(kv, p_lo[j], acc0);
      }
    }
#pragma unroll
    for (int q = 0; q < NF; ++q) {
      vec_t khi, klo;
      magnitude_operands<F16, IL, NK, NF>(ka, q, &khi, &klo);
      acc0 = E::mfma(khi, m_hi[q], acc0);
      acc1 = E::mfma(khi, m_lo[q], acc1);
      acc0 = E::mfma(klo, m_hi[q], acc0);
    }
    return acc0 + acc1;
  };

  for (int sp = 0; sp < kMaxSpans; ++sp) {
    const int tile = tile_first + sp;
    const int t0 = tile * kScoreTile;
    if (t0 >= n) break;  // the same for every wave
    const int t1 = min(n, t0 + kScoreTile);
    const int n_mt = (t1 - t0 + 15) / 16;
    SpanPages pages;
    pages.resolve(kbase, bt, n_blocks, a.num_pages, a.page_stride, t0);

    auto load_tile = [&](int mt, u32x4 (&ka)[NK]) {
      // Unconditional loads of rows inside the pool, as in the mean scorer:
      // tiles past the span re-read its last tile, unresolved pages read page
      // 0, and both are zeroed.
      const int mt_read = mt < n_mt ? mt : n_mt - 1;
      const int rel = mt_read * 16 + r;
      const int t = t0 + rel;
      bool page_ok = false;
      KVC_GLOBAL const uint16_t* pbase = pages.page(rel, &page_ok);
      const bool ok = mt < n_mt && t < t1 && page_ok;
      KVC_GLOBAL const uint16_t* row = pbase + static_cast<int64_t>(t & (kBlockSize - 1)) * row_elems + lane_off;
#pragma unroll
      for (int j = 0; j < NK; ++j) {
        const u32x4 v = load_k(reinterpret_cast<KVC_GLOBAL const u32x4*>(row + 32 * j));
        ka[j] = ok ? v : u32x4{0, 0, 0, 0};
      }
    };

    double sum = 0.0, sumsq = 0.0;
    auto emit = [&](int mt, const f32x4& v) {
      const int rel = mt * 16 + 4 * kb;
      if (writer && mt < n_mt) {
        *reinterpret_cast<f32x4*>(stage_row + rel) = v;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (t0 + rel + i < t1) {
            const double dv = static_cast<double>(v[i]);
            sum += dv;
            sumsq = fma(dv, dv, sumsq);
          }
        }
      }
    };

    // Two tiles per pass over the staged fragments.
    auto score_pair = [&](int mt0, const u32x4 (&k0)[NK], int mt1, const u32x4 (&k1)[NK]) {
      const f32x4 rest0 = rest_tile(k0);
      const f32x4 rest1 = rest_tile(k1);
      f32x4 mx0 = {0.0f, 0.0f, 0.0f, 0.0f}, mx1 = {0.0f, 0.0f, 0.0f, 0.0f};
      for (int gl = 0; gl < gcnt; ++gl) {
        f32x4 best0 = {-INFINITY, -INFINITY, -INFINITY, -INFINITY}, best1 = best0;
        for (int c = 0; c < geo.nch; ++c) {
          const u32x4* wl = lds_frag + ((gl * geo.nch + c) * NR) * 128 + lane;
          f32x4 acc0 = {0.0f, 0.0f, 0.0f, 0.0f};
          f32x4 acc1 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
          for (int st = 0; st < NR; ++st) {
            const vec_t whi = __builtin_bit_cast(vec_t, wl[st * 128]);
            const vec_t wlo = __builtin_bit_cast(vec_t, wl[st * 128 + 64]);
            const vec_t x0 = __builtin_bit_cast(vec_t, k0[st]);
            const vec_t x1 = __builtin_bit_cast(vec_t, k1[st]);
            acc0 = E::mfma(x0, whi, acc0);
            acc1 = E::mfma(x1, whi, acc1);
            acc0 = E::mfma(x0, wlo, acc0);
            acc1 = E::mfma(x1, wlo, acc1);
          }
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            best0[i] = max_nan(best0[i], acc0[i]);
            best1[i] = max_nan(best1[i], acc1[i]);
          }
        }
        const bool mine = r == g0 + gl;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float v0 = row16_max(best0[i]);
          const float v1 = row16_max(best1[i]);
          mx0[i] = mine ? v0 : mx0[i];
          mx1[i] = mine ? v1 : mx1[i];
        }
      }
      f32x4 out0, out1;
      if (F16) {
        out0 = mx0 * o_scale + rest0 * r_scale;
        out1 = mx1 * o_scale + rest1 * r_scale;
      } else {
        out0 = mx0 + rest0;
        out1 = mx1 + rest1;
      }
      emit(mt0, out0);
      emit(mt1, out1);
    };

    // Wave w scores tiles w, w+4, w+8, ... in pairs (w, w+4), (w+8, w+12);
    // the next pair's keys are in flight while the current pair is scored.
    constexpr int kStreams = kScoreThreads / 64;
    u32x4 ka[2][NK], kn[2][NK];
    int mt = wave;
    load_tile(mt, ka[0]);
    load_tile(mt + kStreams, ka[1]);
    for (; mt < n_mt; mt += 4 * kStreams) {
      load_tile(mt + 2 * kStreams, kn[0]);
      load_tile(mt + 3 * kStreams, kn[1]);
      score_pair(mt, ka[0], mt + kStreams, ka[1]);
      if (mt + 2 * kStreams >= n_mt) break;
      load_tile(mt + 4 * kStreams, ka[0]);
      load_tile(mt + 5 * kStreams, ka[1]);
      score_pair(mt + 2 * kStreams, kn[0], mt + 3 * kStreams, kn[1]);
    }

    red[0][threadIdx.x] = sum;
    red[1][threadIdx.x] = sumsq;
    __syncthreads();

    // Stage -> raw scores (rows g0 .. g0+gcnt-1 of this KV head), as the mean scorer.
    const int span = t1 - t0;
    const int q_first = head * qpk + g0;
    if (a.raw_token_stride == 1) {
      const int span4 = (span + 3) >> 2;
      for (int idx = threadIdx.x; idx < gcnt * span4; idx += kScoreThreads) {
        const int row = idx / span4;
        const int c = (idx - row * span4) << 2;
        const float* src = stage + row * kStageStride + c;
        float* dst = raw_out + (tok_base + t0 + c) + static_cast<int64_t>(q_first + row) * a.raw_head_stride;
        if (c + 3 < span && (reinterpret_cast<uintptr_t>(dst) & 15) == 0) {
          __builtin_nontemporal_store(*reinterpret_cast<const f32x4*>(src), reinterpret_cast<f32x4*>(dst));
        } else {
          for (int i = 0; i < 4 && c + i < span; ++i) dst[i] = src[i];
        }
      }
    } else {
      for (int idx = threadIdx.x; idx < gcnt * span; idx += kScoreThreads) {
        const int t = idx / gcnt;
        const int row = idx - t * gcnt;
        raw_out[(tok_base + t0 + t) * a.raw_token_stride + static_cast<int64_t>(q_first + row) * a.raw_head_stride] =
            stage[row * kStageStride + t];
      }
    }
    // Partial sums of query head g: lanes 16k + g of the four waves.
    for (int i = threadIdx.x; i < gcnt; i += kScoreThreads) {
      const int g = g0 + i;
      double s0 = 0.0, s1 = 0.0;
      for (int w = 0; w < kStreams; ++w) {
        for (int k = 0; k < 4; ++k) {
          s0 += red[0][w * 64 + k * 16 + g];
          s1 += red[1][w * 64 + k * 16 + g];
        }
      }
      const int n_heads = a.kv_heads * qpk;
      double* dst = a.partials +
                    (((static_cast<int64_t>(layer) * a.n_seq + b) * a.max_tiles + tile) * n_heads + head * qpk + g) * 2;
      dst[0] = s0;
      dst[1] = s1;
    }
    __syncthreads();  // stage and red are reused by the next span
  }
}

using MaxKernel = void (*)(ScoreArgs, MaxGeometry, int, const u32x4*, const float*, const u32x4*, const float*);

template <bool F16, bool IL>
MaxKernel pick_max_typed(int nk, int nf) {
  switch (nk * 16 + nf) {
    case 2 * 16 + 1: return score_max_kernel<2, 1, F16, IL>;
    case 4 * 16 + 1: return score_max_kernel<4, 1, F16, IL>;
    case 4 * 16 + 2: return score_max_kernel<4, 2, F16, IL>;
    case 8 * 16 + 1: return score_max_kernel<8, 1, F16, IL>;
    case 8 * 16 + 2: return score_max_kernel<8, 2, F16, IL>;
    case 8 * 16 + 4: return score_max_kernel<8, 4, F16, IL>;
    default: return nullptr;
  }
}

}  // namespace

int launch_max_scorer(hipStream_t stream, const ScoreShape& s, int dtype, int n_offsets, const FoldArgs& fa,
                      const ScoreArgs& sa, void* workspace) {
  const int nk = s.head_dim / 32, nf = s.freq / 32, nr = 2 * nf;
  const bool f16 = dtype == KVC_DTYPE_FP16;
  MaxKernel kern = f16 ? (fa.interleaved ? pick_max_typed<true, true>(nk, nf) : pick_max_typed<true, false>(nk, nf))
                       : (fa.interleaved ? pick_max_typed<false, true>(nk, nf) : pick_max_typed<false, false>(nk, nf));
  if (!kern) return fail(KVC_EINVAL, "kvc_score_paged_max: no scorer for head_dim %d rotary_dim %d", s.head_dim, s.rotary_dim);
  MaxGeometry geo;
  geo.nch = offset_chunks(n_offsets);
  const int per_g = geo.nch * nr * 2 * kOffsetFragBytes;
  int gpg = kMaxFragLds / per_g;
  if (gpg < 1)
    return fail(KVC_EINVAL, "kvc_score_paged_max: %d offsets need %d bytes of fragments per query head (limit %d)",
                n_offsets, per_g, kMaxFragLds);
  if (gpg > s.qpk) gpg = s.qpk;
  geo.groups = (s.qpk + gpg - 1) / gpg;
  geo.gpg = (s.qpk + geo.groups - 1) / geo.groups;
  const int64_t items = ceil_div(s.max_tiles, kMaxSpans) * s.kv_heads;
  const int64_t gx = ceil_div(items, 8) * 8 * geo.groups;
  if (gx > 0x7fffffff) return fail(KVC_EINVAL, "kvc_score_paged_max: grid too large");
  geo.work = static_cast<int>(items);

  FoldArgs rest = fa;
  rest.zero_rotary = 1;
  if (int rc = launch_mfma_fold(stream, s, dtype, rest, workspace)) return rc;
  char* tail = static_cast<char*>(workspace) + max_tail_offset(s);
  OffsetFoldArgs m;
  m.f = fa;
  m.n_offsets = n_offsets;
  m.nch = geo.nch;
  m.nr = nr;
  m.frags = reinterpret_cast<u32x4*>(tail);
  m.inv_scale = reinterpret_cast<float*>(tail + (offset_fragment_bytes(s, n_offsets) + 255) / 256 * 256);
  const int64_t cols = static_cast<int64_t>(s.n_seq) * s.n_layers * s.kv_heads * s.qpk;
  if (f16)
    fold_offsets_kernel<true><<<static_cast<unsigned>(ceil_div(cols, 4)), 256, 0, stream>>>(m);
  else
    fold_offsets_kernel<false><<<static_cast<unsigned>(ceil_div(cols, 4)), 256, 0, stream>>>(m);
  if (int rc = launch_status("kvc_score_paged_max(fold)")) return rc;

  const float* rest_scale =
      reinterpret_cast<const float*>(static_cast<const char*>(workspace) + mfma_fragment_only_bytes(s));
  const size_t lds = static_cast<size_t>(geo.gpg) * per_g;
  dim3 grid(static_cast<unsigned>(gx), static_cast<unsigned>(s.n_seq), static_cast<unsigned>(s.n_layers));
  kern<<<grid, kScoreThreads, lds, stream>>>(sa, geo, s.qpk, static_cast<const u32x4*>(workspace), rest_scale, m.frags,
                                             m.inv_scale);
  return launch_status("kvc_score_paged_max");
}

}  // namespace kvc
