// TriAttention paged-K scoring on the matrix cores (v_mfma_f32_16x16x32_bf16).
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
// Work split: a wave owns one KV head and walks 16-token tiles of its
// workgroup's 256-token span; a workgroup covers hpw KV heads (hpw in {1,2,4}
// dividing kv_heads) and 4/hpw interleaved tile streams per head.  The next
// tile's keys are loaded before the current tile's MFMAs.  Raw scores and the
// float64 per-tile partial sums have the same layout as the VALU scorer's, so
// kvc_head_stats and kvc_aggregate are shared.

#include "score_internal.h"

#ifndef KVC_MFMA_GROUP
#define KVC_MFMA_GROUP 2  // 16-token tiles per prefetch group
#endif

namespace kvc {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Two floats -> packed bf16 pair, round to nearest even (one v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
}

// K is read once per scoring layer.  Non-temporal loads (meant to keep K from
// evicting the weight fragments in L2) measured 0.85 ms against 0.72 ms for
// plain loads on the Qwen2.5-14B shape, so they are off by default.
#ifndef KVC_SCORE_NT_K
#define KVC_SCORE_NT_K 0
#endif
__device__ __forceinline__ u32x4 load_k(KVC_GLOBAL const u32x4* p) {
  if (KVC_SCORE_NT_K) return __builtin_nontemporal_load(p);
  return *p;
}

// Round-to-nearest-even float32 -> bf16 bits (finite inputs).
__device__ __forceinline__ uint32_t bf16_bits(float x) {
  const uint32_t u = __float_as_uint(x);
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}
__device__ __forceinline__ float bf16_value(uint32_t bits) { return __uint_as_float(bits << 16); }

constexpr int kMfmaMaxHeadsPerWg = 4;            // hpw
constexpr int kMfmaMaxQpk = 8;                   // make_shape admits qpk <= 8
constexpr int kStageStride = kScoreTile + 4;     // floats per staged query-head row

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
  const float* pc = a.phase_cos + b * a.phase_seq_stride + static_cast<int64_t>(layer) * a.freq;
  const float* ps = a.phase_sin + b * a.phase_seq_stride + static_cast<int64_t>(layer) * a.freq;
  const int head_dim = a.rotary_dim + a.pass;
  const bool low = (frag & 1) != 0;
  const int step = frag >> 1;
  uint16_t out[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float w = 0.0f;
    if (step < nk) {
      const int d = 32 * step + 8 * kb + e;
      if (d < head_dim) {
        if (d < 2 * a.freq) {
          const int f = d < a.freq ? d : d - a.freq;
          const int64_t o = row * a.freq + f;
          const float qr = a.q_real[o], qi = a.q_imag[o], sc = a.scale[o];
          const float c = pc[f], sn = ps[f];
          w = d < a.freq ? sc * (qr * c - qi * sn) : sc * (qi * c + qr * sn);
        } else {
          w = a.q_pass[row * a.pass + (d - a.rotary_dim)];
        }
      }
    } else {
      const int f = 32 * (step - nk) + 8 * kb + e;
      const int64_t o = row * a.freq + f;
      w = a.scale[o] * a.extra[o];
    }
    const uint32_t hi = bf16_bits(w);
    out[e] = static_cast<uint16_t>(low ? bf16_bits(w - bf16_value(hi)) : hi);
  }
  uint16_t* dst = frags + (((((static_cast<int64_t>(b) * a.n_layers + layer) * a.kv_heads + head) * n_frag + frag) * packed) + pl) * 8;
#pragma unroll
  for (int e = 0; e < 8; ++e) dst[e] = out[e];
}

// --------------------------------------------------------------- score ------

template <int NK, int NF>
__global__ __launch_bounds__(kScoreThreads) void score_mfma_kernel(ScoreArgs a, MfmaGeometry geo, int qpk,
                                                                   const u32x4* __restrict__ frags) {
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
    return __builtin_bit_cast(bf16x8, live_col ? v : u32x4{0, 0, 0, 0});
  };
  bf16x8 w_hi[NK], w_lo[NK], m_hi[NF], m_lo[NF];
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
      const bf16x8 kv = __builtin_bit_cast(bf16x8, ka[j]);
      if (j & 1) {
        acc1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kv, w_hi[j], acc1, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kv, w_lo[j], acc1, 0, 0, 0);
      } else {
        acc0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kv, w_hi[j], acc0, 0, 0, 0);
        acc0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kv, w_lo[j], acc0, 0, 0, 0);
      }
    }
#pragma unroll
    for (int q = 0; q < NF; ++q) {
      u32x4 hi, lo;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const uint32_t re_w = ka[q][w], im_w = ka[q + NF][w];
        const float re0 = bf16_lo(re_w), re1 = bf16_hi(re_w);
        const float im0 = bf16_lo(im_w), im1 = bf16_hi(im_w);
        const float m0 = __builtin_amdgcn_sqrtf(fmaf(im0, im0, re0 * re0));
        const float m1 = __builtin_amdgcn_sqrtf(fmaf(im1, im1, re1 * re1));
        const uint32_t h = pack_bf16(m0, m1);
        hi[w] = h;
        lo[w] = pack_bf16(m0 - bf16_lo(h), m1 - bf16_hi(h));
      }
      const bf16x8 khi = __builtin_bit_cast(bf16x8, hi);
      const bf16x8 klo = __builtin_bit_cast(bf16x8, lo);
      acc0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(khi, m_hi[q], acc0, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(khi, m_lo[q], acc1, 0, 0, 0);
      acc0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(klo, m_hi[q], acc0, 0, 0, 0);
    }
    const f32x4 acc = acc0 + acc1;
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

  // Tiles sub, sub + nsub, ... in groups of KVC_MFMA_GROUP; the next group's
  // keys are in flight while the current group is scored.
  constexpr int G = KVC_MFMA_GROUP;
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

using MfmaKernel = void (*)(ScoreArgs, MfmaGeometry, int, const u32x4*);

MfmaKernel pick(int nk, int nf) {
  switch (nk * 16 + nf) {
    case 2 * 16 + 1: return score_mfma_kernel<2, 1>;
    case 4 * 16 + 1: return score_mfma_kernel<4, 1>;
    case 4 * 16 + 2: return score_mfma_kernel<4, 2>;
    case 8 * 16 + 1: return score_mfma_kernel<8, 1>;
    case 8 * 16 + 2: return score_mfma_kernel<8, 2>;
    case 8 * 16 + 4: return score_mfma_kernel<8, 4>;
    default: return nullptr;
  }
}

}  // namespace

bool mfma_scorer_supported(const ScoreShape& s, int dtype, int rope_style) {
  if (dtype != KVC_DTYPE_BF16 || rope_style != KVC_ROPE_HALF) return false;
  if (s.head_dim % 32 != 0 || s.freq % 32 != 0 || s.qpk > kMfmaMaxQpk) return false;
  return pick(s.head_dim / 32, s.freq / 32) != nullptr;
}

int launch_mfma_scorer(hipStream_t stream, const ScoreShape& s, const FoldArgs& fa, const ScoreArgs& sa,
                       void* weights) {
  const MfmaGeometry geo = geometry(s);
  MfmaKernel kern = pick(geo.nk, geo.nf);
  if (!kern) return fail(KVC_EINVAL, "kvc_score_paged: no MFMA scorer for head_dim %d rotary_dim %d", s.head_dim, s.rotary_dim);
  const int64_t fold_threads = static_cast<int64_t>(s.n_seq) * s.n_layers * s.kv_heads * (2 * geo.nk + 2 * geo.nf) * 4 * s.qpk;
  fold_mfma_kernel<<<static_cast<unsigned>(ceil_div(fold_threads, 256)), 256, 0, stream>>>(
      fa, geo.nk, geo.nf, static_cast<uint16_t*>(weights));
  if (int rc = launch_status("kvc_score_paged(fold)")) return rc;
  const int64_t gx = static_cast<int64_t>(s.max_tiles) * geo.head_groups;
  if (gx > 0x7fffffff) return fail(KVC_EINVAL, "kvc_score_paged: grid too large");
  dim3 grid(static_cast<unsigned>(gx), static_cast<unsigned>(s.n_seq), static_cast<unsigned>(s.n_layers));
  kern<<<grid, kScoreThreads, 0, stream>>>(sa, geo, s.qpk, static_cast<const u32x4*>(weights));
  return launch_status("kvc_score_paged");
}

}  // namespace kvc
