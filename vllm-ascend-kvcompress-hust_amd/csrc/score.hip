// TriAttention paged-K scoring on CDNA4.
//
// Kernels:
//   mean_phases_kernel      phase table cos/sin means per (sequence, layer, freq)
//   shift_phases_kernel     the reference device path's angle-addition table
//   fold_weights_kernel     folds calibration stats and phases into per-lane weights
//   score_paged_kernel      reads K once through the block table, writes raw scores
//                           and per-tile float64 partial sums for the head statistics
//   head_stats_kernel       combines the partials into population mean / variance
//   aggregate_kernel        z-normalise, max over heads, combine across layers
//
// Score algebra (tri/scoring.py:66-119).  With a = sqrt(freq_scale_sq), phase
// means c_f, s_f and extra = q_abs - |q_mean|, the score of a post-RoPE key is
//   sum_f a[(qr kr + qi ki) c - (qi kr - qr ki) s] + a*extra*|k_f|  + q_pass.k_pass
// = sum_f kr*W1 + ki*W2 + |k_f|*W3                                  + q_pass.k_pass
// with W1 = a(qr c - qi s), W2 = a(qi c + qr s), W3 = a*extra.  The fold happens
// once per (sequence, layer) so the per-token work is three FMAs per frequency
// per query head, and K is read once per KV head for the whole GQA group.
//
// Lane layout of score_paged_kernel.  A "unit" is two 16-byte chunks of one
// head row: for a rotary unit the 8 real and the 8 imaginary components of 8
// frequencies (half style: dims [8u,8u+8) and [F+8u,F+8u+8); interleaved:
// dims [16u,16u+16)), for a pass unit 16 consecutive unrotated dims.  The
// units of one head row form a lane group of `group` lanes (a power of two);
// a wave holds 64/group groups, each bound to a fixed KV head, so the weights
// stay in registers and every wave load instruction covers whole 128-byte
// lines of consecutive head rows.  Partial dot products are summed across the
// group with DPP, and lane g of the group writes query head g of its KV head.

#include <math.h>
#include <stdarg.h>

#include "score_internal.h"

namespace kvc {
namespace {

// ------------------------------------------------------------- phase tables --

// One group of `width` lanes (the offset count rounded up to a power of two,
// at most 32) per (sequence, layer, frequency); lane o evaluates offset o (then
// o + width, ...), so a thread waits for one cosine/sine instead of one per
// offset.  The phase argument is formed exactly as the torch path does in
// float32, (offset + round_start) * omega, and its cosine/sine are evaluated in
// double and rounded once, so the table agrees with a correctly rounded float32
// evaluation.  Lane 0 of the group sums the rounded values sequentially in
// offset order in float32 and divides by the offset count, as the torch path's
// mean over the offset axis.
constexpr int kPhaseMaxLanes = 32;

__global__ __launch_bounds__(256) void mean_phases_kernel(int n_seq, int n_layers, int n_freq, int width,
                                                          const int64_t* __restrict__ round_starts,
                                                          const float* __restrict__ offsets, int n_offsets,
                                                          const float* __restrict__ omega, float* __restrict__ phase_cos,
                                                          float* __restrict__ phase_sin) {
  const int64_t idx = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) / width;
  const int lane = threadIdx.x & (width - 1);
  const int64_t per_seq = static_cast<int64_t>(n_layers) * n_freq;
  if (idx >= per_seq * n_seq) return;  // the whole lane group leaves together
  const int64_t b = idx / per_seq;
  const int64_t lf = idx - b * per_seq;
  const float rs = static_cast<float>(round_starts[b]);
  const float w = omega[lf];
  float c = 0.0f, s = 0.0f;
  for (int o0 = 0; o0 < n_offsets; o0 += width) {
    const int o = o0 + lane;
    float co = 0.0f, so = 0.0f;
    if (o < n_offsets) {
      const float x = __fmul_rn(__fadd_rn(offsets[o], rs), w);
      co = static_cast<float>(cos(static_cast<double>(x)));
      so = static_cast<float>(sin(static_cast<double>(x)));
    }
    const int count = min(width, n_offsets - o0);
    for (int j = 0; j < count; ++j) {
      c = __fadd_rn(c, __shfl(co, j, width));
      s = __fadd_rn(s, __shfl(so, j, width));
    }
  }
  if (lane == 0) {
    const float n = static_cast<float>(n_offsets);
    phase_cos[idx] = __fdiv_rn(c, n);
    phase_sin[idx] = __fdiv_rn(s, n);
  }
}

// One thread per (sequence, layer, offset, frequency): cos and sin of the
// float32 phase argument (offset + round_start) * omega, as the torch path
// forms it, evaluated in double and rounded once.  Layout [b][l][o][f].
__global__ void offset_phases_kernel(int n_seq, int n_layers, int n_freq, const int64_t* __restrict__ round_starts,
                                     const float* __restrict__ offsets, int n_offsets, const float* __restrict__ omega,
                                     float* __restrict__ phase_cos, float* __restrict__ phase_sin) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t per_layer = static_cast<int64_t>(n_offsets) * n_freq;
  const int64_t per_seq = per_layer * n_layers;
  if (idx >= per_seq * n_seq) return;
  const int64_t b = idx / per_seq;
  const int64_t r = idx - b * per_seq;
  const int64_t l = r / per_layer;
  const int64_t of = r - l * per_layer;
  const int o = static_cast<int>(of / n_freq);
  const int f = static_cast<int>(of - static_cast<int64_t>(o) * n_freq);
  const float rs = static_cast<float>(round_starts[b]);
  const float x = __fmul_rn(__fadd_rn(offsets[o], rs), omega[l * n_freq + f]);
  phase_cos[idx] = static_cast<float>(cos(static_cast<double>(x)));
  phase_sin[idx] = static_cast<float>(sin(static_cast<double>(x)));
}

// Angle addition from precomputed offset means (tri/kernels.py:70-82).
__global__ void shift_phases_kernel(int n_values, float round_start,
                                    const float* __restrict__ omega,
                                    const float* __restrict__ offset_cos,
                                    const float* __restrict__ offset_sin,
                                    float* __restrict__ phase_cos, float* __restrict__ phase_sin) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n_values) return;
  const float x = __fmul_rn(round_start, omega[i]);
  const float rc = static_cast<float>(cos(static_cast<double>(x)));
  const float rsn = static_cast<float>(sin(static_cast<double>(x)));
  const float oc = offset_cos[i], os = offset_sin[i];
  phase_cos[i] = __fsub_rn(__fmul_rn(rc, oc), __fmul_rn(rsn, os));
  phase_sin[i] = __fadd_rn(__fmul_rn(rsn, oc), __fmul_rn(rc, os));
}

// ------------------------------------------------------------- weight fold --



// Weights are laid out in the element order of the lane's two 16-byte chunks
// (chunk a -> W1[0..8), chunk b -> W2[0..8)), so the scorer unpacks both RoPE
// layouts the same way; W3[j] multiplies |k| of frequency 8u+j.
//   half:        a = re[8u..8u+8), b = im[8u..8u+8)
//   interleaved: a = (re,im) of freqs 8u..8u+4, b = (re,im) of freqs 8u+4..8u+8
__global__ void fold_weights_kernel(FoldArgs a) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t total = static_cast<int64_t>(a.n_seq) * a.n_layers * a.kv_heads * a.units;
  if (idx >= total) return;
  const int unit = static_cast<int>(idx % a.units);
  int64_t r = idx / a.units;
  const int head = static_cast<int>(r % a.kv_heads);
  r /= a.kv_heads;
  const int layer = static_cast<int>(r % a.n_layers);
  const int b = static_cast<int>(r / a.n_layers);
  float* out = a.weights + idx * 3 * a.qpk * 8;
  const int64_t stat_row = (static_cast<int64_t>(layer) * a.kv_heads + head) * a.qpk;
  if (unit < a.units_rot) {
    const float* pc = a.phase_cos + b * a.phase_seq_stride + static_cast<int64_t>(layer) * a.freq;
    const float* ps = a.phase_sin + b * a.phase_seq_stride + static_cast<int64_t>(layer) * a.freq;
    for (int g = 0; g < a.qpk; ++g) {
      const int64_t base = (stat_row + g) * a.freq;
      float w_re[8], w_im[8];
      for (int j = 0; j < 8; ++j) {
        const int f = unit * 8 + j;
        const float qr = a.q_real[base + f], qi = a.q_imag[base + f];
        const float sc = a.scale[base + f];
        const float c = pc[f], s = ps[f];
        w_re[j] = sc * (qr * c - qi * s);
        w_im[j] = sc * (qi * c + qr * s);
        out[(2 * a.qpk + g) * 8 + j] = sc * a.extra[base + f];
      }
      for (int e = 0; e < 8; ++e) {
        float w1, w2;
        if (a.interleaved) {
          w1 = (e & 1) ? w_im[e >> 1] : w_re[e >> 1];
          w2 = (e & 1) ? w_im[4 + (e >> 1)] : w_re[4 + (e >> 1)];
        } else {
          w1 = w_re[e];
          w2 = w_im[e];
        }
        out[(0 * a.qpk + g) * 8 + e] = w1;
        out[(1 * a.qpk + g) * 8 + e] = w2;
      }
    }
  } else {
    const int u = unit - a.units_rot;
    for (int g = 0; g < a.qpk; ++g) {
      const float* qp = a.q_pass + (stat_row + g) * a.pass + u * 16;
      for (int j = 0; j < 8; ++j) {
        out[(0 * a.qpk + g) * 8 + j] = qp[j];
        out[(1 * a.qpk + g) * 8 + j] = qp[8 + j];
        out[(2 * a.qpk + g) * 8 + j] = 0.0f;
      }
    }
  }
}

// ----------------------------------------------------------------- scoring --



typedef uint32_t w128 __attribute__((ext_vector_type(4)));

// Sum over aligned groups of GS lanes; every lane of a group ends with the
// same bits (pairwise sums in the same association on every lane).
template <int GS>
__device__ __forceinline__ float group_sum_c(float v) {
  if constexpr (GS >= 2) v += dpp_quad_xor1(v);
  if constexpr (GS >= 4) v += dpp_quad_xor2(v);
  if constexpr (GS >= 8) v += dpp_row_half_mirror(v);
  if constexpr (GS >= 16) v += dpp_row_mirror(v);
  if constexpr (GS >= 32) v += __shfl_xor(v, 16);
  if constexpr (GS >= 64) v += __shfl_xor(v, 32);
  return v;
}

template <typename Tag, int QPK, bool INTERLEAVED, int GS>
__global__ __launch_bounds__(kScoreThreads) void score_paged_kernel(ScoreArgs a) {
  constexpr int kGroupsPerWave = 64 / GS;
  const int layer = blockIdx.z;
  const int b = blockIdx.y;
  const int tile = blockIdx.x;
  const int n = a.seq_lens[b];
  const int t0 = tile * kScoreTile;
  if (t0 >= n) return;  // whole workgroup leaves together
  const int t1 = min(n, t0 + kScoreTile);

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int unit = lane & (GS - 1);
  const int gid = wave * kGroupsPerWave + lane / GS;
  const int n_groups = (kScoreThreads / 64) * kGroupsPerWave;
  const int head = gid % a.kv_heads;
  const int tslot = gid / a.kv_heads;
  const int tpi = n_groups / a.kv_heads;  // tokens per iteration of the workgroup
  const bool active = unit < a.units && tslot < tpi;
  const bool rotary = unit < a.units_rot;

  // Per-lane folded weights for (sequence, layer, head, unit).
  float w1[QPK][8], w2[QPK][8], w3[QPK][8];
  if (active) {
    const float4* wp = reinterpret_cast<const float4*>(
        a.weights +
        ((((static_cast<int64_t>(b) * a.n_layers + layer) * a.kv_heads + head) * a.units + unit) *
         3 * QPK * 8));
#pragma unroll
    for (int g = 0; g < QPK; ++g) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const float4 v1 = wp[(0 * QPK + g) * 2 + h];
        const float4 v2 = wp[(1 * QPK + g) * 2 + h];
        const float4 v3 = wp[(2 * QPK + g) * 2 + h];
        w1[g][4 * h + 0] = v1.x; w1[g][4 * h + 1] = v1.y; w1[g][4 * h + 2] = v1.z; w1[g][4 * h + 3] = v1.w;
        w2[g][4 * h + 0] = v2.x; w2[g][4 * h + 1] = v2.y; w2[g][4 * h + 2] = v2.z; w2[g][4 * h + 3] = v2.w;
        w3[g][4 * h + 0] = v3.x; w3[g][4 * h + 1] = v3.y; w3[g][4 * h + 2] = v3.z; w3[g][4 * h + 3] = v3.w;
      }
    }
  } else {
#pragma unroll
    for (int g = 0; g < QPK; ++g)
#pragma unroll
      for (int j = 0; j < 8; ++j) w1[g][j] = w2[g][j] = w3[g][j] = 0.0f;
  }

  // Element offsets of the lane's two chunks inside the head row.
  int d1, d2;
  if (rotary) {
    if (INTERLEAVED) {
      d1 = 16 * unit;
      d2 = d1 + 8;
    } else {
      d1 = 8 * unit;
      d2 = a.freq + 8 * unit;
    }
  } else {
    d1 = a.rotary_dim + 16 * (unit - a.units_rot);
    d2 = d1 + 8;
  }

  KVC_GLOBAL const uint16_t* kbase = gptr_from_int<const uint16_t>(a.k_layer_ptrs[layer]);
  const int64_t* bt = a.block_ids + a.block_offsets[b];
  const int64_t n_blocks = a.block_offsets[b + 1] - a.block_offsets[b];
  const int64_t row_elems = static_cast<int64_t>(a.kv_heads) * a.head_dim;
  const int64_t head_off = static_cast<int64_t>(head) * a.head_dim;
  const int64_t tok_base = a.token_offsets[b];
  float* raw_out = a.raw + layer * a.raw_layer_stride;
  const bool writer = unit < QPK && tslot < tpi;
  const int q_head = head * QPK + unit;
  const int iters = (t1 - t0 + tpi - 1) / tpi;

  // Token group k (kUnroll iterations) <-> registers: loads are issued one
  // group ahead of the arithmetic that consumes them.
  SpanPages pages;
  pages.resolve(kbase, bt, n_blocks, a.num_pages, a.page_stride, t0);

  auto load_group = [&](int k0, w128 (&ca)[kUnroll], w128 (&cb)[kUnroll]) {
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int k = k0 + u;
      const int t = t0 + tslot + k * tpi;
      // Unconditional loads from a row inside the pool (see the matrix-core
      // scorer): iterations the prefetch reaches past the span re-read the
      // last iteration's rows (cache hits), lanes without a unit read offset 0,
      // and both are zeroed.
      const bool live = k < iters && t < t1 && active;
      const int t_read = t0 + tslot + (k < iters ? k : iters - 1) * tpi;
      bool page_ok = false;
      KVC_GLOBAL const uint16_t* pbase = pages.page(t_read < t1 ? t_read - t0 : 0, &page_ok);
      KVC_GLOBAL const uint16_t* row = pbase + static_cast<int64_t>(t_read & (kBlockSize - 1)) * row_elems + head_off;
      const w128 va = *reinterpret_cast<KVC_GLOBAL const w128*>(row + (active ? d1 : 0));
      const w128 vb = *reinterpret_cast<KVC_GLOBAL const w128*>(row + (active ? d2 : 0));
      const bool ok = live && page_ok;
      ca[u] = ok ? va : w128{0, 0, 0, 0};
      cb[u] = ok ? vb : w128{0, 0, 0, 0};
    }
  };

  double sum = 0.0, sumsq = 0.0;
  auto compute_group = [&](int k0, const w128 (&ca)[kUnroll], const w128 (&cb)[kUnroll]) {
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int k = k0 + u;
      const int t = t0 + tslot + k * tpi;
      float x1[8], x2[8], x3[8];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        x1[2 * j] = Unpack<Tag>::lo(ca[u][j]);
        x1[2 * j + 1] = Unpack<Tag>::hi(ca[u][j]);
        x2[2 * j] = Unpack<Tag>::lo(cb[u][j]);
        x2[2 * j + 1] = Unpack<Tag>::hi(cb[u][j]);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        float re, im;
        if (INTERLEAVED) {
          re = j < 4 ? x1[2 * j] : x2[2 * (j - 4)];
          im = j < 4 ? x1[2 * j + 1] : x2[2 * (j - 4) + 1];
        } else {
          re = x1[j];
          im = x2[j];
        }
        const float m = __builtin_amdgcn_sqrtf(fmaf(im, im, re * re));
        x3[j] = rotary ? m : 0.0f;
      }
      float acc[QPK];
#pragma unroll
      for (int g = 0; g < QPK; ++g) {
        float v = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          v = fmaf(w1[g][j], x1[j], v);
          v = fmaf(w2[g][j], x2[j], v);
          v = fmaf(w3[g][j], x3[j], v);
        }
        acc[g] = group_sum_c<GS>(v);
      }
      float mine = acc[0];
#pragma unroll
      for (int g = 1; g < QPK; ++g) mine = (unit == g) ? acc[g] : mine;
      if (writer && k < iters && t < t1) {
        raw_out[(tok_base + t) * a.raw_token_stride + q_head * a.raw_head_stride] = mine;
        const double dv = static_cast<double>(mine);
        sum += dv;
        sumsq = fma(dv, dv, sumsq);
      }
    }
  };

  w128 pa[kUnroll], pb[kUnroll], qa[kUnroll], qb[kUnroll];
  load_group(0, pa, pb);
  for (int k0 = 0; k0 < iters; k0 += 2 * kUnroll) {
    load_group(k0 + kUnroll, qa, qb);
    compute_group(k0, pa, pb);
    if (k0 + kUnroll >= iters) break;
    load_group(k0 + 2 * kUnroll, pa, pb);
    compute_group(k0 + kUnroll, qa, qb);
  }

  // Combine the per-lane partial sums of each query head in a fixed order.
  __shared__ double red[2][kScoreThreads];
  red[0][threadIdx.x] = sum;
  red[1][threadIdx.x] = sumsq;
  __syncthreads();
  const int n_heads = a.kv_heads * QPK;
  for (int q = threadIdx.x; q < n_heads; q += kScoreThreads) {
    const int h = q / QPK, g = q - h * QPK;
    double s0 = 0.0, s1 = 0.0;
    for (int slot = 0; slot < tpi; ++slot) {
      const int gg = slot * a.kv_heads + h;  // group bound to head h, token slot `slot`
      const int th = (gg / kGroupsPerWave) * 64 + (gg % kGroupsPerWave) * GS + g;
      s0 += red[0][th];
      s1 += red[1][th];
    }
    double* dst = a.partials +
                  (((static_cast<int64_t>(layer) * a.n_seq + b) * a.max_tiles + tile) * n_heads + q) * 2;
    dst[0] = s0;
    dst[1] = s1;
  }
}

// --------------------------------------------------------------- head stats --

// One wave per (layer, sequence, query head): lane l sums tiles l, l+64, ...
// and a fixed butterfly combines the lanes, so the result is the same on
// every run.  Population variance as torch.var_mean(correction=0).
__global__ __launch_bounds__(256) void head_stats_kernel(int n_layers, int n_seq, int n_heads, int max_tiles,
                                                         const int32_t* __restrict__ seq_lens,
                                                         const double* __restrict__ partials,
                                                         float* __restrict__ mean, float* __restrict__ var) {
  const int64_t idx = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) >> 6;
  const int lane = threadIdx.x & 63;
  if (idx >= static_cast<int64_t>(n_layers) * n_seq * n_heads) return;  // whole wave leaves together
  const int q = static_cast<int>(idx % n_heads);
  const int64_t ls = idx / n_heads;  // layer * n_seq + b
  const int b = static_cast<int>(ls % n_seq);
  const int n = seq_lens[b];
  const int tiles = static_cast<int>((n + kScoreTile - 1) / kScoreTile);
  double s0 = 0.0, s1 = 0.0;
  for (int t = lane; t < tiles; t += 64) {
    const double* p = partials + ((ls * max_tiles + t) * n_heads + q) * 2;
    s0 += p[0];
    s1 += p[1];
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    s0 += __shfl_xor(s0, off);
    s1 += __shfl_xor(s1, off);
  }
  if (lane != 0) return;
  const double inv_n = 1.0 / static_cast<double>(n);
  const double m = s0 * inv_n;
  double v = s1 * inv_n - m * m;
  if (v < 0.0) v = 0.0;
  mean[idx] = static_cast<float>(m);
  var[idx] = static_cast<float>(v);
}

// ---------------------------------------------------------------- aggregate --

constexpr int kAggThreads = 256;
constexpr int kAggMaxStats = 4096;  // layers * heads staged in LDS

struct AggArgs {
  int n_layers, n_heads, n_seq, layer_mode;
  unsigned flags;
  const int32_t* seq_lens;
  const int64_t* token_offsets;
  const float* raw;
  int64_t raw_layer_stride, raw_token_stride, raw_head_stride;
  const float* mean;
  const float* var;
  int64_t stats_layer_stride, stats_seq_stride;
  float* agg;
  int64_t layer_out_stride;  // 0: combine layers into agg; else layer l's head maxima at agg + l*stride
};

__device__ __forceinline__ float normalise(float s, float mean, float scale, bool rsqrt_form) {
  return rsqrt_form ? (s - mean) * scale : (s - mean) / scale;
}

__device__ __forceinline__ float combine_layers(float total, float best, int l, const AggArgs& a,
                                                int64_t tok) {
  if (l == 0) {
    if (a.flags & KVC_AGG_ACCUMULATE) {
      const float prev = a.agg[tok];
      return (a.layer_mode == KVC_LAYER_MEAN) ? prev + best : max_nan(prev, best);
    }
    return best;
  }
  return (a.layer_mode == KVC_LAYER_MEAN) ? total + best : max_nan(total, best);
}

__device__ __forceinline__ float finalize_total(float total, unsigned flags, int layer_mode, int n_layers) {
  if (flags & KVC_AGG_FINALIZE) {
    if (layer_mode == KVC_LAYER_MEAN) total = total / static_cast<float>(n_layers);
    if (total != total) total = -INFINITY;
    else if (total == INFINITY) total = 1e30f;
  }
  return total;
}

__device__ __forceinline__ float finalize(float total, const AggArgs& a) {
  return finalize_total(total, a.flags, a.layer_mode, a.n_layers);
}

__device__ void load_layer_stats(const AggArgs& a, int b, float* s_mean, float* s_scale) {
  const int n_stats = a.n_layers * a.n_heads;
  const bool rsqrt_form = (a.flags & KVC_AGG_RSQRT) != 0;
  for (int i = threadIdx.x; i < n_stats; i += kAggThreads) {
    const int l = i / a.n_heads, h = i - l * a.n_heads;
    const int64_t si = l * a.stats_layer_stride + b * a.stats_seq_stride + h;
    const float v = fmaxf(a.var[si], 1e-6f);
    s_mean[i] = a.mean[si];
    s_scale[i] = rsqrt_form ? rsqrtf(v) : sqrtf(v);
  }
}

// Four lanes per token: lane q of a token takes heads q, q+4, q+8, ...; the
// four partial maxima meet through two DPP quad permutations.  Per-(layer,
// head) means and scales sit in LDS.  Works for any score strides.
constexpr int kAggLanes = 4;
constexpr int kAggTokensPerBlock = kAggThreads / kAggLanes;

__device__ __forceinline__ float quad_max_nan(float v) {
  v = max_nan(v, dpp_quad_xor1(v));
  v = max_nan(v, dpp_quad_xor2(v));
  return v;
}

__global__ __launch_bounds__(kAggThreads) void aggregate_kernel(AggArgs a) {
  extern __shared__ float dyn[];
  float* s_mean = dyn;
  float* s_scale = dyn + a.n_layers * a.n_heads;
  const int b = blockIdx.y;
  const int n = a.seq_lens[b];
  if (static_cast<int64_t>(blockIdx.x) * kAggTokensPerBlock >= n) return;
  load_layer_stats(a, b, s_mean, s_scale);
  __syncthreads();
  const int t = blockIdx.x * kAggTokensPerBlock + threadIdx.x / kAggLanes;
  const int q = threadIdx.x & (kAggLanes - 1);
  const bool valid = t < n;
  const bool rsqrt_form = (a.flags & KVC_AGG_RSQRT) != 0;
  const int64_t tok = a.token_offsets[b] + (valid ? t : 0);
  float total = 0.0f;
  for (int l = 0; l < a.n_layers; ++l) {
    const float* row = a.raw + l * a.raw_layer_stride + tok * a.raw_token_stride;
    float best = -INFINITY;
    if (valid) {
      for (int h = q; h < a.n_heads; h += kAggLanes) {
        const int i = l * a.n_heads + h;
        best = max_nan(best, normalise(row[h * a.raw_head_stride], s_mean[i], s_scale[i], rsqrt_form));
      }
    }
    best = quad_max_nan(best);
    if (a.layer_out_stride) {
      if (valid && q == 0) a.agg[l * a.layer_out_stride + tok] = best;
      continue;
    }
    total = combine_layers(total, best, l, a, tok);
  }
  if (valid && q == 0 && !a.layer_out_stride) a.agg[tok] = finalize(total, a);
}

// Head-major scores (unit token stride): two lanes per token, the lower and
// upper halves of a wave, each taking every other head (h = part, part + 2,
// ...), so every load of a wave reads 32 consecutive tokens of two heads
// (two 128-byte runs) with eight loads in flight per lane, and the two partial
// maxima meet through one exchange across the halves.  Twice the waves of one
// lane per token: 104 against 112 us on 4 x 131072 tokens x 6 layers x 40
// heads, level on the smaller batches.
constexpr int kAggHeadUnroll = 8;
constexpr int kAggTokLanes = 2;
constexpr int kAggTokPerBlock = kAggThreads / kAggTokLanes;

__global__ __launch_bounds__(kAggThreads) void aggregate_tokens_kernel(AggArgs a) {
  extern __shared__ float dyn[];
  float* s_mean = dyn;
  float* s_scale = dyn + a.n_layers * a.n_heads;
  const int b = blockIdx.y;
  const int n = a.seq_lens[b];
  if (static_cast<int64_t>(blockIdx.x) * kAggTokPerBlock >= n) return;
  load_layer_stats(a, b, s_mean, s_scale);
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int part = lane >> 5;  // which half of the heads
  const int t = blockIdx.x * kAggTokPerBlock + (threadIdx.x >> 6) * 32 + (lane & 31);
  const bool valid = t < n;
  const bool rsqrt_form = (a.flags & KVC_AGG_RSQRT) != 0;
  const int64_t tok = a.token_offsets[b] + (valid ? t : 0);
  float total = 0.0f;
  for (int l = 0; l < a.n_layers; ++l) {
    const float* col = a.raw + l * a.raw_layer_stride + tok;
    const float* lm = s_mean + l * a.n_heads;
    const float* ls = s_scale + l * a.n_heads;
    float best = -INFINITY;
    if (valid) {
      int h = part;
      for (; h + kAggTokLanes * (kAggHeadUnroll - 1) < a.n_heads; h += kAggTokLanes * kAggHeadUnroll) {
        float v[kAggHeadUnroll];
#pragma unroll
        for (int u = 0; u < kAggHeadUnroll; ++u) v[u] = col[(h + kAggTokLanes * u) * a.raw_head_stride];
#pragma unroll
        for (int u = 0; u < kAggHeadUnroll; ++u) {
          const int hh = h + kAggTokLanes * u;
          best = max_nan(best, normalise(v[u], lm[hh], ls[hh], rsqrt_form));
        }
      }
      for (; h < a.n_heads; h += kAggTokLanes)
        best = max_nan(best, normalise(col[h * a.raw_head_stride], lm[h], ls[h], rsqrt_form));
    }
    best = max_nan(best, __shfl_xor(best, 32));
    if (a.layer_out_stride) {
      if (valid && part == 0) a.agg[l * a.layer_out_stride + tok] = best;
      continue;
    }
    total = combine_layers(total, best, l, a, tok);
  }
  if (valid && part == 0 && !a.layer_out_stride) a.agg[tok] = finalize(total, a);
}

// Layer scores [n_layers][stride] -> aggregate: layers combined in layer order
// (copy, then + or NaN-propagating max), as the fused aggregate does.
__global__ void combine_layer_scores_kernel(int n_layers, int64_t n_tokens, const float* __restrict__ layer_scores,
                                            int64_t layer_stride, int layer_mode, unsigned flags, float* agg) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= n_tokens) return;
  float total = 0.0f;
  for (int l = 0; l < n_layers; ++l) {
    const float v = layer_scores[l * layer_stride + t];
    if (l == 0) {
      total = v;
      if (flags & KVC_AGG_ACCUMULATE) total = (layer_mode == KVC_LAYER_MEAN) ? agg[t] + v : max_nan(agg[t], v);
    } else {
      total = (layer_mode == KVC_LAYER_MEAN) ? total + v : max_nan(total, v);
    }
  }
  agg[t] = finalize_total(total, flags, layer_mode, n_layers);
}

using ScoreKernelFn = void (*)(ScoreArgs);

template <typename Tag, bool IL, int GS>
ScoreKernelFn pick_qpk(int qpk) {
  switch (qpk) {
    case 1: return score_paged_kernel<Tag, 1, IL, GS>;
    case 2: return score_paged_kernel<Tag, 2, IL, GS>;
    case 3: return score_paged_kernel<Tag, 3, IL, GS>;
    case 4: return score_paged_kernel<Tag, 4, IL, GS>;
    case 5: return score_paged_kernel<Tag, 5, IL, GS>;
    case 6: return score_paged_kernel<Tag, 6, IL, GS>;
    case 7: return score_paged_kernel<Tag, 7, IL, GS>;
    case 8: return score_paged_kernel<Tag, 8, IL, GS>;
    default: return nullptr;
  }
}

template <typename Tag, bool IL>
ScoreKernelFn pick_group(int shift, int qpk) {
  switch (shift) {
    case 3: return pick_qpk<Tag, IL, 8>(qpk);
    case 4: return pick_qpk<Tag, IL, 16>(qpk);
    case 5: return pick_qpk<Tag, IL, 32>(qpk);
    default: return nullptr;
  }
}

}  // namespace
}  // namespace kvc

using namespace kvc;

extern "C" int kvc_mean_phases(kvc_stream_t stream, int n_seq, int n_layers, int n_freq,
                               const int64_t* round_starts, const float* offsets, int n_offsets,
                               const float* omega, float* phase_cos, float* phase_sin) {
  if (n_seq <= 0 || n_layers <= 0 || n_freq <= 0 || n_offsets <= 0)
    return fail(KVC_EINVAL, "kvc_mean_phases: sizes must be positive");
  if (!round_starts || !offsets || !omega || !phase_cos || !phase_sin)
    return fail(KVC_EINVAL, "kvc_mean_phases: null pointer");
  const int64_t total = static_cast<int64_t>(n_seq) * n_layers * n_freq;
  int width = 1;
  while (width < n_offsets && width < kPhaseMaxLanes) width <<= 1;
  if (ceil_div(total * width, 256) > 0x7fffffff) return fail(KVC_EINVAL, "kvc_mean_phases: grid too large");
  mean_phases_kernel<<<static_cast<unsigned>(ceil_div(total * width, 256)), 256, 0, as_stream(stream)>>>(
      n_seq, n_layers, n_freq, width, round_starts, offsets, n_offsets, omega, phase_cos, phase_sin);
  return launch_status("kvc_mean_phases");
}

extern "C" int kvc_offset_phases(kvc_stream_t stream, int n_seq, int n_layers, int n_freq,
                                 const int64_t* round_starts, const float* offsets, int n_offsets,
                                 const float* omega, float* phase_cos, float* phase_sin) {
  if (n_seq <= 0 || n_layers <= 0 || n_freq <= 0 || n_offsets <= 0)
    return fail(KVC_EINVAL, "kvc_offset_phases: sizes must be positive");
  if (!round_starts || !offsets || !omega || !phase_cos || !phase_sin)
    return fail(KVC_EINVAL, "kvc_offset_phases: null pointer");
  const int64_t total = static_cast<int64_t>(n_seq) * n_layers * n_offsets * n_freq;
  offset_phases_kernel<<<static_cast<unsigned>(ceil_div(total, 256)), 256, 0, as_stream(stream)>>>(
      n_seq, n_layers, n_freq, round_starts, offsets, n_offsets, omega, phase_cos, phase_sin);
  return launch_status("kvc_offset_phases");
}

extern "C" int kvc_shift_mean_phases(kvc_stream_t stream, int n_values, int64_t round_start,
                                     const float* omega, const float* offset_cos_mean,
                                     const float* offset_sin_mean, float* phase_cos,
                                     float* phase_sin) {
  if (n_values <= 0) return fail(KVC_EINVAL, "kvc_shift_mean_phases: n_values must be positive");
  if (!omega || !offset_cos_mean || !offset_sin_mean || !phase_cos || !phase_sin)
    return fail(KVC_EINVAL, "kvc_shift_mean_phases: null pointer");
  shift_phases_kernel<<<static_cast<unsigned>(ceil_div(n_values, 256)), 256, 0,
                        as_stream(stream)>>>(n_values, static_cast<float>(round_start), omega,
                                             offset_cos_mean, offset_sin_mean, phase_cos,
                                             phase_sin);
  return launch_status("kvc_shift_mean_phases");
}

extern "C" size_t kvc_score_workspace_bytes(int n_layers, int kv_heads, int head_dim,
                                            int rotary_dim, int qpk, int n_seq, int max_seq_len) {
  ScoreShape s;
  if (!make_shape(&s, n_layers, kv_heads, head_dim, rotary_dim, qpk, n_seq, max_seq_len)) return 0;
  return workspace_bytes(s);
}

extern "C" int kvc_score_raw_layout(int dtype, int rope_style, int kv_heads, int head_dim, int rotary_dim,
                                    int qpk) {
  ScoreShape s;
  if (!make_shape(&s, 1, kv_heads, head_dim, rotary_dim, qpk, 1, 0))
    return fail(KVC_EINVAL, "kvc_score_raw_layout: unsupported shape");
  if (dtype != KVC_DTYPE_BF16 && dtype != KVC_DTYPE_FP16)
    return fail(KVC_EINVAL, "kvc_score_raw_layout: dtype must be bf16 or fp16");
  if (rope_style != KVC_ROPE_HALF && rope_style != KVC_ROPE_INTERLEAVED)
    return fail(KVC_EINVAL, "kvc_score_raw_layout: unknown rope style %d", rope_style);
  return mfma_scorer_supported(s, dtype, rope_style) ? KVC_RAW_HEAD_MAJOR : KVC_RAW_TOKEN_MAJOR;
}

namespace kvc {
namespace {

// Checks and argument blocks shared by kvc_score_paged and kvc_score_paged_max.
// `phase_bytes_ok` is false when the caller's phase tables cannot be read by
// this entry (checked by the caller).  Returns 0 or a C-ABI error code.
int score_setup(const char* who, int dtype, int n_layers, const uint64_t* k_layer_ptrs, int64_t num_pages,
                int64_t page_stride, int kv_heads, int head_dim, int rotary_dim, int qpk, int rope_style, int n_seq,
                int max_seq_len, const int32_t* seq_lens, const int64_t* token_offsets, const int64_t* block_offsets,
                const int64_t* block_ids, const float* q_real, const float* q_imag, const float* freq_scale,
                const float* extra_coef, const float* q_pass, const float* phase_cos, const float* phase_sin,
                int64_t phase_seq_stride, float* raw, int64_t raw_layer_stride, int64_t raw_token_stride,
                int64_t raw_head_stride, void* workspace, size_t workspace_bytes_given, size_t workspace_needed,
                ScoreShape* s, FoldArgs* fa, ScoreArgs* sa) {
  if (!make_shape(s, n_layers, kv_heads, head_dim, rotary_dim, qpk, n_seq, max_seq_len))
    return fail(KVC_EINVAL,
                "%s: unsupported shape (layers=%d kv_heads=%d head_dim=%d "
                "rotary_dim=%d qpk=%d n_seq=%d); rotary_dim and head_dim-rotary_dim must be "
                "multiples of 16, qpk <= 8",
                who, n_layers, kv_heads, head_dim, rotary_dim, qpk, n_seq);
  if (dtype != KVC_DTYPE_BF16 && dtype != KVC_DTYPE_FP16)
    return fail(KVC_EINVAL, "%s: dtype must be bf16 or fp16", who);
  if (rope_style != KVC_ROPE_HALF && rope_style != KVC_ROPE_INTERLEAVED)
    return fail(KVC_EINVAL, "%s: unknown rope style %d", who, rope_style);
  if (page_stride < static_cast<int64_t>(kBlockSize) * kv_heads * head_dim || num_pages <= 0)
    return fail(KVC_EINVAL, "%s: page stride smaller than a page", who);
  if (!k_layer_ptrs || !seq_lens || !token_offsets || !block_offsets || !block_ids || !q_real ||
      !q_imag || !freq_scale || !extra_coef || !phase_cos || !phase_sin || !raw || !workspace)
    return fail(KVC_EINVAL, "%s: null pointer", who);
  if (s->pass > 0 && !q_pass)
    return fail(KVC_EINVAL, "%s: partial RoPE requires q_pass", who);
  if (workspace_bytes_given < workspace_needed)
    return fail(KVC_EINVAL, "%s: workspace too small (%zu < %zu)", who, workspace_bytes_given, workspace_needed);

  fa->n_seq = n_seq;
  fa->n_layers = n_layers;
  fa->kv_heads = kv_heads;
  fa->qpk = qpk;
  fa->freq = s->freq;
  fa->pass = s->pass;
  fa->units_rot = s->units_rot;
  fa->units = s->units;
  fa->rotary_dim = rotary_dim;
  fa->interleaved = rope_style == KVC_ROPE_INTERLEAVED ? 1 : 0;
  fa->zero_rotary = 0;
  fa->q_real = q_real;
  fa->q_imag = q_imag;
  fa->scale = freq_scale;
  fa->extra = extra_coef;
  fa->q_pass = q_pass;
  fa->phase_cos = phase_cos;
  fa->phase_sin = phase_sin;
  fa->phase_seq_stride = phase_seq_stride;
  fa->weights = static_cast<float*>(workspace);

  sa->k_layer_ptrs = k_layer_ptrs;
  sa->num_pages = num_pages;
  sa->page_stride = page_stride;
  sa->kv_heads = kv_heads;
  sa->head_dim = head_dim;
  sa->rotary_dim = rotary_dim;
  sa->freq = s->freq;
  sa->units_rot = s->units_rot;
  sa->units = s->units;
  sa->group_shift = s->group_shift;
  sa->n_seq = n_seq;
  sa->max_tiles = s->max_tiles;
  sa->n_layers = n_layers;
  sa->seq_lens = seq_lens;
  sa->token_offsets = token_offsets;
  sa->block_offsets = block_offsets;
  sa->block_ids = block_ids;
  sa->weights = static_cast<float*>(workspace);
  sa->raw = raw;
  sa->raw_layer_stride = raw_layer_stride;
  sa->raw_token_stride = raw_token_stride;
  sa->raw_head_stride = raw_head_stride;
  sa->partials = reinterpret_cast<double*>(static_cast<char*>(workspace) + weights_bytes_aligned(*s));
  return 0;
}

}  // namespace
}  // namespace kvc

extern "C" int kvc_score_paged(kvc_stream_t stream, int dtype, int n_layers,
                               const uint64_t* k_layer_ptrs, int64_t num_pages,
                               int64_t page_stride, int kv_heads, int head_dim, int rotary_dim,
                               int qpk, int rope_style, int n_seq, int max_seq_len,
                               const int32_t* seq_lens, const int64_t* token_offsets,
                               const int64_t* block_offsets, const int64_t* block_ids,
                               const float* q_real, const float* q_imag, const float* freq_scale,
                               const float* extra_coef, const float* q_pass,
                               const float* phase_cos, const float* phase_sin,
                               int64_t phase_seq_stride, float* raw, int64_t raw_layer_stride,
                               int64_t raw_token_stride, int64_t raw_head_stride, void* workspace,
                               size_t workspace_bytes_given) {
  ScoreShape s;
  FoldArgs fa;
  ScoreArgs sa;
  const size_t need = make_shape(&s, n_layers, kv_heads, head_dim, rotary_dim, qpk, n_seq, max_seq_len)
                          ? workspace_bytes(s)
                          : 0;
  if (int rc = score_setup("kvc_score_paged", dtype, n_layers, k_layer_ptrs, num_pages, page_stride, kv_heads,
                           head_dim, rotary_dim, qpk, rope_style, n_seq, max_seq_len, seq_lens, token_offsets,
                           block_offsets, block_ids, q_real, q_imag, freq_scale, extra_coef, q_pass, phase_cos,
                           phase_sin, phase_seq_stride, raw, raw_layer_stride, raw_token_stride, raw_head_stride,
                           workspace, workspace_bytes_given, need, &s, &fa, &sa))
    return rc;
  if (s.max_tiles == 0) return 0;
  hipStream_t st = as_stream(stream);

  if (mfma_scorer_supported(s, dtype, rope_style)) return launch_mfma_scorer(st, s, dtype, fa, sa, workspace);

  const int64_t fold_threads = static_cast<int64_t>(n_seq) * n_layers * kv_heads * s.units;
  fold_weights_kernel<<<static_cast<unsigned>(ceil_div(fold_threads, 64)), 64, 0, st>>>(fa);
  if (int rc = launch_status("kvc_score_paged(fold)")) return rc;

  ScoreKernelFn kern = nullptr;
  const bool il = rope_style == KVC_ROPE_INTERLEAVED;
  const int gs = s.group_shift;
  if (dtype == KVC_DTYPE_BF16)
    kern = il ? pick_group<Bf16Tag, true>(gs, qpk) : pick_group<Bf16Tag, false>(gs, qpk);
  else
    kern = il ? pick_group<Fp16Tag, true>(gs, qpk) : pick_group<Fp16Tag, false>(gs, qpk);
  if (!kern) return fail(KVC_EINVAL, "kvc_score_paged: qpk %d unsupported", qpk);
  dim3 grid(static_cast<unsigned>(s.max_tiles), static_cast<unsigned>(n_seq),
            static_cast<unsigned>(n_layers));
  if (n_seq > 65535 || n_layers > 65535)
    return fail(KVC_EINVAL, "kvc_score_paged: too many sequences or layers for one launch");
  kern<<<grid, kScoreThreads, 0, st>>>(sa);
  return launch_status("kvc_score_paged");
}

extern "C" size_t kvc_score_max_workspace_bytes(int n_layers, int kv_heads, int head_dim, int rotary_dim, int qpk,
                                                int n_seq, int max_seq_len, int n_offsets) {
  ScoreShape s;
  if (n_offsets <= 0 || !make_shape(&s, n_layers, kv_heads, head_dim, rotary_dim, qpk, n_seq, max_seq_len)) return 0;
  return max_workspace_bytes(s, n_offsets);
}

extern "C" int kvc_score_paged_max(kvc_stream_t stream, int dtype, int n_layers, const uint64_t* k_layer_ptrs,
                                   int64_t num_pages, int64_t page_stride, int kv_heads, int head_dim,
                                   int rotary_dim, int qpk, int rope_style, int n_seq, int max_seq_len,
                                   const int32_t* seq_lens, const int64_t* token_offsets,
                                   const int64_t* block_offsets, const int64_t* block_ids, const float* q_real,
                                   const float* q_imag, const float* freq_scale, const float* extra_coef,
                                   const float* q_pass, const float* offset_cos, const float* offset_sin,
                                   int n_offsets, int64_t phase_seq_stride, float* raw, int64_t raw_layer_stride,
                                   int64_t raw_token_stride, int64_t raw_head_stride, void* workspace,
                                   size_t workspace_bytes_given) {
  ScoreShape s;
  FoldArgs fa;
  ScoreArgs sa;
  if (n_offsets <= 0) return fail(KVC_EINVAL, "kvc_score_paged_max: n_offsets must be positive");
  const size_t need = make_shape(&s, n_layers, kv_heads, head_dim, rotary_dim, qpk, n_seq, max_seq_len)
                          ? max_workspace_bytes(s, n_offsets)
                          : 0;
  if (int rc = score_setup("kvc_score_paged_max", dtype, n_layers, k_layer_ptrs, num_pages, page_stride, kv_heads,
                           head_dim, rotary_dim, qpk, rope_style, n_seq, max_seq_len, seq_lens, token_offsets,
                           block_offsets, block_ids, q_real, q_imag, freq_scale, extra_coef, q_pass, offset_cos,
                           offset_sin, phase_seq_stride, raw, raw_layer_stride, raw_token_stride, raw_head_stride,
                           workspace, workspace_bytes_given, need, &s, &fa, &sa))
    return rc;
  if (phase_seq_stride != 0 && phase_seq_stride < static_cast<int64_t>(n_layers) * n_offsets * s.freq)
    return fail(KVC_EINVAL, "kvc_score_paged_max: phase_seq_stride smaller than one sequence's table");
  if (s.max_tiles == 0) return 0;
  if (n_seq > 65535 || n_layers > 65535)
    return fail(KVC_EINVAL, "kvc_score_paged_max: too many sequences or layers for one launch");
  return launch_max_scorer(as_stream(stream), s, dtype, n_offsets, fa, sa, workspace);
}

extern "C" int kvc_head_stats(kvc_stream_t stream, int n_layers, int kv_heads, int head_dim,
                              int rotary_dim, int qpk, int n_seq, int max_seq_len,
                              const int32_t* seq_lens, const void* workspace,
                              size_t workspace_bytes_given, float* mean, float* var) {
  ScoreShape s;
  if (!make_shape(&s, n_layers, kv_heads, head_dim, rotary_dim, qpk, n_seq, max_seq_len))
    return fail(KVC_EINVAL, "kvc_head_stats: unsupported shape");
  if (!seq_lens || !workspace || !mean || !var)
    return fail(KVC_EINVAL, "kvc_head_stats: null pointer");
  if (workspace_bytes_given < workspace_bytes(s))
    return fail(KVC_EINVAL, "kvc_head_stats: workspace too small");
  const double* partials = reinterpret_cast<const double*>(
      static_cast<const char*>(workspace) + weights_bytes_aligned(s));
  const int n_heads = kv_heads * qpk;
  const int64_t total = static_cast<int64_t>(n_layers) * n_seq * n_heads;
  head_stats_kernel<<<static_cast<unsigned>(ceil_div(total * 64, 256)), 256, 0, as_stream(stream)>>>(
      n_layers, n_seq, n_heads, s.max_tiles > 0 ? s.max_tiles : 1, seq_lens, partials, mean, var);
  return launch_status("kvc_head_stats");
}

namespace kvc {
namespace {

int launch_aggregate(const char* who, kvc_stream_t stream, int n_layers, int n_heads, int n_seq, int max_seq_len,
                     const int32_t* seq_lens, const int64_t* token_offsets, const float* raw,
                     int64_t raw_layer_stride, int64_t raw_token_stride, int64_t raw_head_stride, const float* mean,
                     const float* var, int64_t stats_layer_stride, int64_t stats_seq_stride, int layer_aggregation,
                     unsigned flags, float* out, int64_t layer_out_stride) {
  if (n_layers <= 0 || n_heads <= 0 || n_seq <= 0 || max_seq_len < 0)
    return fail(KVC_EINVAL, "%s: sizes must be positive", who);
  if (n_layers * n_heads > kAggMaxStats)
    return fail(KVC_EINVAL, "%s: layers*heads %d exceeds %d", who, n_layers * n_heads, kAggMaxStats);
  if (layer_aggregation != KVC_LAYER_MEAN && layer_aggregation != KVC_LAYER_MAX)
    return fail(KVC_EINVAL, "%s: unknown layer aggregation %d", who, layer_aggregation);
  if (!seq_lens || !token_offsets || !raw || !mean || !var || !out) return fail(KVC_EINVAL, "%s: null pointer", who);
  if (n_seq > 65535) return fail(KVC_EINVAL, "%s: too many sequences", who);
  if (max_seq_len == 0) return 0;
  AggArgs aa;
  aa.n_layers = n_layers;
  aa.n_heads = n_heads;
  aa.n_seq = n_seq;
  aa.layer_mode = layer_aggregation;
  aa.flags = flags;
  aa.seq_lens = seq_lens;
  aa.token_offsets = token_offsets;
  aa.raw = raw;
  aa.raw_layer_stride = raw_layer_stride;
  aa.raw_token_stride = raw_token_stride;
  aa.raw_head_stride = raw_head_stride;
  aa.mean = mean;
  aa.var = var;
  aa.stats_layer_stride = stats_layer_stride;
  aa.stats_seq_stride = stats_seq_stride;
  aa.agg = out;
  aa.layer_out_stride = layer_out_stride;
  const size_t lds = static_cast<size_t>(2) * n_layers * n_heads * sizeof(float);
  if (raw_token_stride == 1) {
    dim3 grid(static_cast<unsigned>(ceil_div(max_seq_len, kAggTokPerBlock)), static_cast<unsigned>(n_seq));
    aggregate_tokens_kernel<<<grid, kAggThreads, lds, as_stream(stream)>>>(aa);
    return launch_status(who);
  }
  dim3 grid(static_cast<unsigned>(ceil_div(max_seq_len, kAggTokensPerBlock)), static_cast<unsigned>(n_seq));
  aggregate_kernel<<<grid, kAggThreads, lds, as_stream(stream)>>>(aa);
  return launch_status(who);
}

}  // namespace
}  // namespace kvc

extern "C" int kvc_aggregate(kvc_stream_t stream, int n_layers, int n_heads, int n_seq,
                             int max_seq_len, const int32_t* seq_lens,
                             const int64_t* token_offsets, const float* raw,
                             int64_t raw_layer_stride, int64_t raw_token_stride,
                             int64_t raw_head_stride, const float* mean, const float* var,
                             int64_t stats_layer_stride, int64_t stats_seq_stride,
                             int layer_aggregation, unsigned flags, float* agg) {
  return launch_aggregate("kvc_aggregate", stream, n_layers, n_heads, n_seq, max_seq_len, seq_lens, token_offsets,
                          raw, raw_layer_stride, raw_token_stride, raw_head_stride, mean, var, stats_layer_stride,
                          stats_seq_stride, layer_aggregation, flags, agg, 0);
}

extern "C" int kvc_layer_head_max(kvc_stream_t stream, int n_layers, int n_heads, int n_seq, int max_seq_len,
                                  const int32_t* seq_lens, const int64_t* token_offsets, const float* raw,
                                  int64_t raw_layer_stride, int64_t raw_token_stride, int64_t raw_head_stride,
                                  const float* mean, const float* var, int64_t stats_layer_stride,
                                  int64_t stats_seq_stride, unsigned flags, float* layer_scores,
                                  int64_t layer_stride) {
  if (layer_stride <= 0) return fail(KVC_EINVAL, "kvc_layer_head_max: layer_stride must be positive");
  return launch_aggregate("kvc_layer_head_max", stream, n_layers, n_heads, n_seq, max_seq_len, seq_lens,
                          token_offsets, raw, raw_layer_stride, raw_token_stride, raw_head_stride, mean, var,
                          stats_layer_stride, stats_seq_stride, KVC_LAYER_MEAN, flags & KVC_AGG_RSQRT, layer_scores,
                          layer_stride);
}

extern "C" int kvc_combine_layer_scores(kvc_stream_t stream, int n_layers, int64_t n_tokens, const float* layer_scores,
                                        int64_t layer_stride, int layer_aggregation, unsigned flags, float* agg) {
  if (n_layers <= 0 || n_tokens < 0 || layer_stride < n_tokens)
    return fail(KVC_EINVAL, "kvc_combine_layer_scores: bad sizes");
  if (layer_aggregation != KVC_LAYER_MEAN && layer_aggregation != KVC_LAYER_MAX)
    return fail(KVC_EINVAL, "kvc_combine_layer_scores: unknown layer aggregation %d", layer_aggregation);
  if (n_tokens == 0) return 0;
  if (!layer_scores || !agg) return fail(KVC_EINVAL, "kvc_combine_layer_scores: null pointer");
  combine_layer_scores_kernel<<<static_cast<unsigned>(ceil_div(n_tokens, 256)), 256, 0, as_stream(stream)>>>(
      n_layers, n_tokens, layer_scores, layer_stride, layer_aggregation, flags, agg);
  return launch_status("kvc_combine_layer_scores");
}
