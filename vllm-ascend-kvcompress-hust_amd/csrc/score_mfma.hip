// TriAttention paged-K scoring on the matrix cores (v_mfma_f32_16x16x32_bf16 /
// v_mfma_f32_16x16x32_f16).
//
// The linear part of the score is a small GEMM per KV head: a 16-token x
// head_dim tile of bf16 keys times head_dim x 16 folded weights (query heads of
// the GQA group on the N axis, unused columns zero).  The keys are exact bf16
// A operands read straight from the paged cache; the float32 weights enter as a
// bf16 hi/lo pair (W = hi + lo to ~2^-16), so two MFMAs per 32-deep K step
// give the float32 dot product to well inside the parity tolerance.  The
// magnitude term sum_f W3_f |k_f| is a second GEMM over the F frequencies with
// |k| computed in the lane (hi/lo split as well; hi*hi + hi*lo + lo*hi).
//
// Operand layout of v_mfma_f32_16x16x32_bf16 (checked on the device): lane l
// holds A[l%16][8*(l/16) + e], B[8*(l/16) + e][l%16] and D[4*(l/16) + i][l%16].
// K step j of the linear part covers head dims 32j .. 32j+31, so lane l of
// step j reads dims 32j + 8*(l/16) .. +8 of token l%16: one 16-byte load.  With
// half-style RoPE and F a multiple of 32, the real parts (step j < F/32) and
// imaginary parts (step j + F/32) of frequencies 32j + 8*(l/16) + e sit in the
// same lane, so |k| needs no data exchange and lands exactly in the layout of
// the magnitude GEMM's A operand.
//
// Interleaved RoPE keeps (real, imaginary) of frequency f in dims (2f, 2f+1),
// so each 32-bit word of a lane's K chunk is one frequency: linear steps 2q and
// 2q+1 give the lane 4 + 4 magnitudes, frequencies 16(2q+h) + 4*(l/16) + i for
// h in {0,1}, i < 4, which fill magnitude step q (the fold lays the magnitude
// weights out in the same order), again without a data exchange.
//
// fp16 caches: the keys are exact fp16 A operands and the weights enter as
// fp16 hi/lo pairs (about 22 significant bits).  fp16's range is narrow, so
// each query head's weights (a B column) are first scaled by a power of two
// that brings the column's largest weight to [2^13, 2^14); the column of the
// product is scaled back on the float32 accumulator, both steps exact.  |k| is
// scaled by 1/4 before its fp16 split (|k| of fp16 keys can exceed 65504) and
// the magnitude weights by 4.
//
// Work split: a wave owns one KV head and walks 16-token tiles of its
// workgroup's 256-token span; a workgroup covers hpw KV heads (hpw in {1,2,4}
// dividing kv_heads) and 4/hpw interleaved tile streams per head.  The next
// tile's keys are loaded before the current tile's MFMAs.  Raw scores and the
// float64 per-tile partial sums have the same layout as the VALU scorer's, so
// kvc_head_stats and kvc_aggregate are shared.

#include "mfma_common.h"


namespace kvc {
namespace {

constexpr int kMfmaMaxHeadsPerWg = 4;            // hpw

struct MfmaGeometry {
  int nk, nf;         // linear / magnitude K steps of 32
  int hpw, nsub;      // KV heads per workgroup, tile streams per head
  int head_groups;    // kv_heads / hpw
};

inline MfmaGeometry geometry(const ScoreShape& s) {
  MfmaGeometry g;
  g.nk = s.head_dim / 32;
  g.nf = s.freq / 32;
  g.hpw = (s.kv_heads % 4 == 0) ? 4 : (s.kv_heads % 2 == 0) ? 2 : 1;
  g.nsub = 4 / g.hpw;
  g.head_groups = s.kv_heads / g.hpw;
  return g;
}

// ---------------------------------------------------------------- fold ------

// One thread per (sequence, layer, KV head, fragment, live lane): the lane's
// eight bf16 values of one fragment.  Only the lanes of live query heads
// (g < qpk) are stored, packed as [fragment][kb][g]; the scorer zeroes the
// B columns of the other lanes, so a wave reads qpk/16 of a full fragment.  Linear weight of head dim d for query head g
// (tri/scoring.py:70-81, 117-119 folded with the phase means):
//   d <  F      : sqrt(fss) (qr c - qi s)     (real part, frequency d)
//   F <= d < 2F : sqrt(fss) (qi c + qr s)     (imaginary part, frequency d-F)
//   d >= R      : q_pass[d - R]
// Magnitude weight of frequency f: sqrt(fss) * extra.  Fragments 2j / 2j+1
// hold the hi / lo bf16 parts of linear step j, 2nk+2q / 2nk+2q+1 those of
// magnitude step q.
// Folded weight of K-step element (step, kb, e) for query head g of
// (sequence b, layer, KV head): see fold_mfma_kernel.
__device__ __forceinline__ float folded_weight(const FoldArgs& a, int nk, int b, int layer, int64_t row, int step,
                                              int kb, int e) {
  const int head_dim = a.rotary_dim + a.pass;
  if (step < nk) {
    const int d = 32 * step + 8 * kb + e;
    if (d >= head_dim) return 0.0f;
    if (d < 2 * a.freq) {
      if (a.zero_rotary) return 0.0f;
      const float* pc = a.phase_cos + b * a.phase_seq_stride + static_cast<int64_t>(layer) * a.freq;
      const float* ps = a.phase_sin + b * a.phase_seq_stride + static_cast<int64_t>(layer) * a.freq;
      // Half style: real parts in dims [0, F), imaginary in [F, 2F); interleaved: (2f, 2f+1).
      const bool real = a.interleaved ? (d & 1) == 0 : d < a.freq;
      const int f = a.interleaved ? d >> 1 : (d < a.freq ? d : d - a.freq);
      const int64_t o = row * a.freq + f;
      const float qr = a.q_real[o], qi = a.q_imag[o], sc = a.scale[o];
      const float c = pc[f], sn = ps[f];
      return real ? sc * (qr * c - qi * sn) : sc * (qi * c + qr * sn);
    }
    return a.q_pass[row * a.pass + (d - a.rotary_dim)];
  }
  const int q = step - nk;
  const int f = a.interleaved ? 16 * (2 * q + (e >> 2)) + 4 * kb + (e & 3) : 32 * q + 8 * kb + e;
  const int64_t o = row * a.freq + f;
  return a.scale[o] * a.extra[o];
}

__global__ void fold_mfma_kernel(FoldArgs a, int nk, int nf, uint16_t* __restrict__ frags) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int n_frag = 2 * nk + 2 * nf;
  const int packed = 4 * a.qpk;  // live lanes per fragment
  const int64_t total = static_cast<int64_t>(a.n_seq) * a.n_layers * a.kv_heads * n_frag * packed;
  if (idx >= total) return;
  const int pl = static_cast<int>(idx % packed);
  int64_t r = idx / packed;
  const int frag = static_cast<int>(r % n_frag);
  r /= n_frag;
  const int head = static_cast<int>(r % a.kv_heads);
  r /= a.kv_heads;
  const int layer = static_cast<int>(r % a.n_layers);
  const int b = static_cast<int>(r / a.n_layers);
  const int g = pl % a.qpk;
  const int kb = pl / a.qpk;
  const int64_t row = ((static_cast<int64_t>(layer) * a.kv_heads + head) * a.qpk + g);
  const bool low = (frag & 1) != 0;
  const int step = frag >> 1;
  uint16_t out[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float w = folded_weight(a, nk, b, layer, row, step, kb, e);
    const uint32_t hi = bf16_bits(w);
    out[e] = static_cast<uint16_t>(low ? bf16_bits(w - bf16_value(hi)) : hi);
  }
  uint16_t* dst = frags + (((((static_cast<int64_t>(b) * a.n_layers + layer) * a.kv_heads + head) * n_frag + frag) * packed) + pl) * 8;
#pragma unroll
  for (int e = 0; e < 8; ++e) dst[e] = out[e];
}

// fp16 fragments: one wave per (sequence, layer, KV head, query head g), 256
// threads per workgroup.  Lane l < 4*(nk+nf) owns K step l/4, row block l%4:
// its eight weights (magnitude weights times 1/kMagScale), then the column's
// largest magnitude over the wave picks the power-of-two scale 2^s that brings
// it to [2^13, 2^14) (s in [-126, 126]; none when it is 0, inf or NaN).  The
// lane writes fp16(2^s w) and fp16(2^s w - hi) to fragments 2 step and
// 2 step + 1 in the packed layout of fold_mfma_kernel; lane 0 writes 2^-s.
__global__ __launch_bounds__(256) void fold_mfma_f16_kernel(FoldArgs a, int nk, int nf, uint16_t* __restrict__ frags,
                                                            float* __restrict__ inv_scale) {
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
  const int64_t row = ((static_cast<int64_t>(layer) * a.kv_heads + head) * a.qpk + g);
  const bool active = lane < 4 * (nk + nf);
  const int step = lane >> 2, kb = lane & 3;
  float w[8];
  float big = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    w[e] = active ? folded_weight(a, nk, b, layer, row, step, kb, e) : 0.0f;
    if (step >= nk) w[e] *= 1.0f / MfmaElem<true>::kMagScale;
    big = fmaxf(big, fabsf(w[e]));
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) big = fmaxf(big, __shfl_xor(big, off));
  int sh = 0;
  if (big > 0.0f && big <= 3.4e38f) {
    int ex;
    (void)frexpf(big, &ex);  // big < 2^ex
    sh = 14 - ex;
    sh = sh < -126 ? -126 : (sh > 126 ? 126 : sh);
  }
  if (active) {
    const int n_frag = 2 * nk + 2 * nf;
    const int packed = 4 * a.qpk;
    const int64_t base = (((static_cast<int64_t>(b) * a.n_layers + layer) * a.kv_heads + head) * n_frag + 2 * step) * packed +
                         kb * a.qpk + g;
    uint16_t hi[8], lo[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float v = ldexpf(w[e], sh);
      const _Float16 h = static_cast<_Float16>(v);
      hi[e] = __builtin_bit_cast(uint16_t, h);
      lo[e] = __builtin_bit_cast(uint16_t, static_cast<_Float16>(v - static_cast<float>(h)));
    }
    uint16_t* dhi = frags + base * 8;
    uint16_t* dlo = frags + (base + packed) * 8;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      dhi[e] = hi[e];
      dlo[e] = lo[e];
    }
  }
  if (lane == 0) inv_scale[col] = ldexpf(1.0f, -sh);
}

// --------------------------------------------------------------- score ------

template <int NK, int NF, bool F16, bool IL>
__global__ __launch_bounds__(kScoreThreads) void score_mfma_kernel(ScoreArgs a, MfmaGeometry geo, int qpk,
                                                                   const u32x4* __restrict__ frags,
                                                                   const float* __restrict__ inv_scale) {
  typedef MfmaElem<F16> E;
  typedef typename E::vec vec_t;
  const int layer = blockIdx.z;
  const int b = blockIdx.y;
  const int tile = blockIdx.x / geo.head_groups;
  const int hg = blockIdx.x - tile * geo.head_groups;
  const int n = a.seq_lens[b];
  const int t0 = tile * kScoreTile;
  if (t0 >= n) return;  // whole workgroup leaves together
  const int t1 = min(n, t0 + kScoreTile);

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r = lane & 15;   // A row (token in tile) / D column (query head)
  const int kb = lane >> 4;  // K block of A/B, row block of D
  const int head = hg * geo.hpw + wave % geo.hpw;
  const int sub = wave / geo.hpw;

  // Folded weight fragments of (sequence, layer, head).
  constexpr int kFrags = 2 * NK + 2 * NF;
  // Packed fragments [frag][kb][g < qpk]; lanes of query heads g >= qpk read
  // the kb group's first word (a line the live lanes read anyway) and zero it.
  const int packed = 4 * qpk;
  const bool live_col = r < qpk;
  const u32x4* fp = frags + (((static_cast<int64_t>(b) * a.n_layers + layer) * a.kv_heads + head) * kFrags) * packed +
                    kb * qpk + (live_col ? r : 0);
  auto frag_word = [&](int f) {
    const u32x4 v = fp[f * packed];
    return __builtin_bit_cast(vec_t, live_col ? v : u32x4{0, 0, 0, 0});
  };
  vec_t w_hi[NK], w_lo[NK], m_hi[NF], m_lo[NF];
  // fp16: the scale that takes this lane's output column back from the
  // scaled weights.
  const float col_scale =
      F16 ? inv_scale[((static_cast<int64_t>(b) * a.n_layers + layer) * a.kv_heads + head) * qpk + (live_col ? r : 0)]
          : 1.0f;
#pragma unroll
  for (int j = 0; j < NK; ++j) {
    w_hi[j] = frag_word(2 * j);
    w_lo[j] = frag_word(2 * j + 1);
  }
#pragma unroll
  for (int q = 0; q < NF; ++q) {
    m_hi[q] = frag_word(2 * NK + 2 * q);
    m_lo[q] = frag_word(2 * NK + 2 * q + 1);
  }

  KVC_GLOBAL const uint16_t* kbase = gptr_from_int<const uint16_t>(a.k_layer_ptrs[layer]);
  const int64_t* bt = a.block_ids + a.block_offsets[b];
  const int64_t n_blocks = a.block_offsets[b + 1] - a.block_offsets[b];
  const int64_t row_elems = static_cast<int64_t>(a.kv_heads) * a.head_dim;
  const int64_t lane_off = static_cast<int64_t>(head) * a.head_dim + 8 * kb;
  const int64_t tok_base = a.token_offsets[b];
  float* raw_out = a.raw + layer * a.raw_layer_stride;
  const int n_mt = (t1 - t0 + 15) / 16;  // 16-token tiles in the span
  const bool writer = r < qpk;
  const int hl_wave = wave % geo.hpw;  // KV head slot of this wave inside the workgroup

  // Score stage: [hpw][qpk][kStageStride] floats, rows padded by four floats
  // so the query-head rows of one wave start in different LDS banks.
  __shared__ __attribute__((aligned(16))) float stage[kMfmaMaxHeadsPerWg * kMfmaMaxQpk * kStageStride];
  float* stage_row = stage + (hl_wave * qpk + (writer ? r : 0)) * kStageStride;

  SpanPages pages;
  pages.resolve(kbase, bt, n_blocks, a.num_pages, a.page_stride, t0);

  auto load_tile = [&](int mt, u32x4 (&ka)[NK]) {
    // The loads are unconditional (loads under a branch would make the
    // compiler wait for every load in flight at the join) and always hit a row
    // inside the pool: tiles the prefetch reaches past the span re-read the
    // span's last tile, which this wave has just read (a cache hit, not HBM
    // traffic), and unresolved pages read page 0.  Out-of-range rows are zeroed.
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
  auto score_tile = [&](int mt, const u32x4 (&ka)[NK]) {
    // Two independent accumulation chains keep consecutive MFMAs apart.
    f32x4 acc0 = {0.0f, 0.0f, 0.0f, 0.0f};
    f32x4 acc1 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < NK; ++j) {
      const vec_t kv = __builtin_bit_cast(vec_t, ka[j]);
      if (j & 1) {
        acc1 = E::mfma(kv, w_hi[j], acc1);
        acc1 = E::mfma(kv, w_lo[j], acc1);
      } else {
        acc0 = E::mfma(kv, w_hi[j], acc0);
        acc0 = E::mfma(kv, w_lo[j], acc0);
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
    f32x4 acc = acc0 + acc1;
    if (F16) acc *= col_scale;
    // D[4*kb + i][r]: token t0 + 16*mt + 4*kb + i, query head r of this KV head.
    // Scores go to the workgroup's LDS stage (four adjacent tokens per lane,
    // one 16-byte write); global stores wait until the span is done, so the
    // loop's waits cover only K loads (vector memory operations retire in
    // issue order, and a store in the loop would hold up the next tile).
    const int rel = mt * 16 + 4 * kb;
    if (writer && mt < n_mt) {
      *reinterpret_cast<f32x4*>(stage_row + rel) = acc;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (t0 + rel + i < t1) {
          const double dv = static_cast<double>(acc[i]);
          sum += dv;
          sumsq = fma(dv, dv, sumsq);
        }
      }
    }
  };

  // Tiles sub, sub + nsub, ... in groups of G; the next group's
  // keys are in flight while the current group is scored.
  constexpr int G = 2;  // 16-token tiles per prefetch group
  u32x4 ka[G][NK], kb2[G][NK];
  const int step = geo.nsub;
  int mt = sub;
#pragma unroll
  for (int g = 0; g < G; ++g) load_tile(mt + g * step, ka[g]);
  for (; mt < n_mt; mt += 2 * G * step) {
#pragma unroll
    for (int g = 0; g < G; ++g) load_tile(mt + (G + g) * step, kb2[g]);
#pragma unroll
    for (int g = 0; g < G; ++g) score_tile(mt + g * step, ka[g]);
    if (mt + G * step >= n_mt) break;
#pragma unroll
    for (int g = 0; g < G; ++g) load_tile(mt + (2 * G + g) * step, ka[g]);
#pragma unroll
    for (int g = 0; g < G; ++g) score_tile(mt + (G + g) * step, kb2[g]);
  }

  // Per query head: sum the lanes of the four row blocks and the tile streams.
  __shared__ double red[2][kScoreThreads];
  red[0][threadIdx.x] = sum;
  red[1][threadIdx.x] = sumsq;
  __syncthreads();

  // Stage -> raw scores: row (hl, g) holds query head (hg*hpw + hl)*qpk + g
  // for the span's tokens.  Head-major scores are contiguous per row (16-byte
  // stores where aligned); token-major ones are contiguous across the rows.
  // Non-temporal 16-byte stores measured 1-2% faster scoring than plain ones
  // (the scores are read once more, by the aggregation pass).
  const int span = t1 - t0;
  const int rows = geo.hpw * qpk;
  const int q_first = hg * geo.hpw * qpk;
  if (a.raw_token_stride == 1) {
    const int span4 = (span + 3) >> 2;
    for (int idx = threadIdx.x; idx < rows * span4; idx += kScoreThreads) {
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
    for (int idx = threadIdx.x; idx < rows * span; idx += kScoreThreads) {
      const int t = idx / rows;
      const int row = idx - t * rows;
      raw_out[(tok_base + t0 + t) * a.raw_token_stride + static_cast<int64_t>(q_first + row) * a.raw_head_stride] =
          stage[row * kStageStride + t];
    }
  }
  const int heads_here = geo.hpw * qpk;
  for (int i = threadIdx.x; i < heads_here; i += kScoreThreads) {
    const int hl = i / qpk, g = i - hl * qpk;
    double s0 = 0.0, s1 = 0.0;
    for (int sb = 0; sb < geo.nsub; ++sb) {
      const int w = sb * geo.hpw + hl;
      for (int k = 0; k < 4; ++k) {
        s0 += red[0][w * 64 + k * 16 + g];
        s1 += red[1][w * 64 + k * 16 + g];
      }
    }
    const int q = (hg * geo.hpw + hl) * qpk + g;
    const int n_heads = a.kv_heads * qpk;
    double* dst = a.partials + (((static_cast<int64_t>(layer) * a.n_seq + b) * a.max_tiles + tile) * n_heads + q) * 2;
    dst[0] = s0;
    dst[1] = s1;
  }
}

using MfmaKernel = void (*)(ScoreArgs, MfmaGeometry, int, const u32x4*, const float*);

template <bool F16, bool IL>
MfmaKernel pick_typed(int nk, int nf) {
  switch (nk * 16 + nf) {
    case 2 * 16 + 1: return score_mfma_kernel<2, 1, F16, IL>;
    case 4 * 16 + 1: return score_mfma_kernel<4, 1, F16, IL>;
    case 4 * 16 + 2: return score_mfma_kernel<4, 2, F16, IL>;
    case 8 * 16 + 1: return score_mfma_kernel<8, 1, F16, IL>;
    case 8 * 16 + 2: return score_mfma_kernel<8, 2, F16, IL>;
    case 8 * 16 + 4: return score_mfma_kernel<8, 4, F16, IL>;
    default: return nullptr;
  }
}
MfmaKernel pick(int nk, int nf, int dtype, int rope_style) {
  const bool il = rope_style == KVC_ROPE_INTERLEAVED;
  if (dtype == KVC_DTYPE_FP16) return il ? pick_typed<true, true>(nk, nf) : pick_typed<true, false>(nk, nf);
  return il ? pick_typed<false, true>(nk, nf) : pick_typed<false, false>(nk, nf);
}

}  // namespace

bool mfma_scorer_supported(const ScoreShape& s, int dtype, int rope_style) {
  if (dtype != KVC_DTYPE_BF16 && dtype != KVC_DTYPE_FP16) return false;
  if (rope_style != KVC_ROPE_HALF && rope_style != KVC_ROPE_INTERLEAVED) return false;
  if (s.head_dim % 32 != 0 || s.freq % 32 != 0 || s.qpk > kMfmaMaxQpk) return false;
  return pick(s.head_dim / 32, s.freq / 32, dtype, rope_style) != nullptr;
}

int64_t mfma_fold_items(const ScoreShape& s, int dtype) {
  const MfmaGeometry geo = geometry(s);
  const int64_t cols = static_cast<int64_t>(s.n_seq) * s.n_layers * s.kv_heads * s.qpk;
  // fp16: one wave per weight column, four per workgroup; bf16: one thread per
  // live lane of every fragment.
  if (dtype == KVC_DTYPE_FP16) return ceil_div(cols, 4) * 256;
  return ceil_div(cols * (2 * geo.nk + 2 * geo.nf) * 4, 256) * 256;
}

int launch_mfma_fold(hipStream_t stream, const ScoreShape& s, int dtype, const FoldArgs& fa, void* weights) {
  const MfmaGeometry geo = geometry(s);
  const int64_t items = mfma_fold_items(s, dtype);
  if (items > kMaxDispatchItems)
    return fail(KVC_EINVAL, "kvc_score_paged: the weight fold's %lld work-items exceed one dispatch",
                static_cast<long long>(items));
  uint16_t* frags = static_cast<uint16_t*>(weights);
  float* inv_scale = reinterpret_cast<float*>(static_cast<char*>(weights) + mfma_fragment_only_bytes(s));
  const unsigned blocks = static_cast<unsigned>(items / 256);
  if (dtype == KVC_DTYPE_FP16) {
    fold_mfma_f16_kernel<<<blocks, 256, 0, stream>>>(fa, geo.nk, geo.nf, frags, inv_scale);
  } else {
    fold_mfma_kernel<<<blocks, 256, 0, stream>>>(fa, geo.nk, geo.nf, frags);
  }
  return launch_status("kvc_score_paged(fold)");
}

int launch_mfma_scorer(hipStream_t stream, const ScoreShape& s, int dtype, const FoldArgs& fa, const ScoreArgs& sa,
                       void* weights) {
  const MfmaGeometry geo = geometry(s);
  MfmaKernel kern = pick(geo.nk, geo.nf, dtype, fa.interleaved ? KVC_ROPE_INTERLEAVED : KVC_ROPE_HALF);
  if (!kern) return fail(KVC_EINVAL, "kvc_score_paged: no MFMA scorer for head_dim %d rotary_dim %d", s.head_dim, s.rotary_dim);
  if (int rc = launch_mfma_fold(stream, s, dtype, fa, weights)) return rc;
  const uint16_t* frags = static_cast<const uint16_t*>(weights);
  const float* inv_scale = reinterpret_cast<const float*>(static_cast<const char*>(weights) + mfma_fragment_only_bytes(s));
  const int64_t gx = static_cast<int64_t>(s.max_tiles) * geo.head_groups;
  if (gx > 0x7fffffff) return fail(KVC_EINVAL, "kvc_score_paged: grid too large");
  dim3 grid(static_cast<unsigned>(gx), static_cast<unsigned>(s.n_seq), static_cast<unsigned>(s.n_layers));
  kern<<<grid, kScoreThreads, 0, stream>>>(sa, geo, s.qpk, reinterpret_cast<const u32x4*>(frags), inv_scale);
  return launch_status("kvc_score_paged");
}

}  // namespace kvc
