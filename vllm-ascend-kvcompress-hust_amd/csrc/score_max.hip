// TriAttention scores with score_aggregation = "max" on the matrix cores
// (tri/scoring.py:84-97): the rotary term is maximised over the future
// offsets instead of averaged,
//   score = max_o sum_f a[(qr kr + qi ki) cos(phi_of) - (qi kr - qr ki) sin(phi_of)]
//         + sum_f a*extra*|k_f| + q_pass.k_pass,      phi_of = (o + rs) * omega_f.
// For one offset the rotary term is a dot product of the key with per-offset
// folded weights, kr*a(qr c - qi s) + ki*a(qi c + qr s), so every (query
// head, offset) pair is one row of a small GEMM against the keys.  Per query
// head the offsets fill chunks of 16 rows (rows past the last offset repeat
// it, which leaves the maximum unchanged).  The weights are the A operand and
// the keys the B operand of v_mfma_f32_16x16x32_{bf16,f16}; a B operand lane
// holds the same eight key values as an A operand lane of the mean scorer
// (token l%16, dims 8*(l/16)..+8 of the K step), so the key loads are shared.
// D[4*kb + i][t] is then offset 4*kb + i of token t.  The maximum over a
// query head's offsets is taken in two steps: in-lane over the four rows of a
// lane's row block (per head of a quad of four heads), then over the four
// row blocks by one reduce-scatter per quad (two v_permlane32_swap, one
// v_permlane16_swap and three maxima), which leaves head 4*q + kb of quad q
// in row block kb.  The magnitude and pass terms do not depend on the offset:
// they come from the mean scorer's fragments (rotary weights zero) in the
// same transposed form, rows permuted so that D[4*kb + i][t] = query head
// 4*i + kb, the head the reduce-scatter leaves in that lane for quad i, and
// are added after the maximum, as in the reference.
//
// Work split: a workgroup owns one KV head, a group of its query heads (all of
// them when their fragments fit the LDS budget) and kMaxSpans consecutive
// 256-token spans; its four waves walk interleaved 16-token tiles of a span.
// The per-offset fragments (bf16 or fp16 hi/lo, 1 KB per 32 rotary dims and
// chunk) are staged in LDS once per workgroup; each fragment read feeds two
// key tiles (one in the three-waves-per-SIMD form).  Workgroups that share a
// key span but not a query-head group are placed eight apart in the grid, on
// the same XCD, so the second read of the keys is an L2 hit.  Raw scores and partial sums have the mean scorer's
// layout, so kvc_head_stats and kvc_aggregate are shared.

#include <math.h>

#include <type_traits>

#include "mfma_common.h"


namespace kvc {
namespace {

constexpr int kMaxSpans = 4;  // 256-token spans per workgroup
constexpr int kMaxFragLds = 48 * 1024;  // bytes of per-offset fragments staged per workgroup
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
// A-operand lane l of every (chunk, step) fragment: offset row 16*chunk +
// l%16 (clamped to the last offset), rotary dims 32*step + 8*(l/16) + e.  fp16
// weights of a query head are scaled by the power of two that brings the
// largest to [2^13, 2^14), as the mean scorer's fp16 fold does.
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

// Tail chunks: one thread per (sequence, layer, KV head, tail chunk, step,
// operand lane).  Row 4*rb + i of chunk tc holds query head 4*quad + i at
// offset 16 + oi: with two quads of heads a chunk (R <= 2 tail offsets),
// quad = 2*tc + rb/2 and oi = min(rb % 2, R - 1); with one (R = 3, 4),
// quad = tc and oi = min(rb, R - 1).  Heads past the last repeat it (rows
// whose maximum is never stored), as do offsets past the last.
__global__ __launch_bounds__(256) void fold_offsets_tail_bf16_kernel(OffsetFoldArgs m, int tail_r, int tail_qpc,
                                                                     int tail_n, int64_t tail_base) {
  typedef MfmaElem<false> E;
  const FoldArgs& a = m.f;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t items = static_cast<int64_t>(a.n_seq) * a.n_layers * a.kv_heads * tail_n * m.nr * 64;
  if (idx >= items) return;
  const int lane = static_cast<int>(idx & 63);
  const int st = static_cast<int>((idx >> 6) % m.nr);
  int64_t r = (idx >> 6) / m.nr;
  const int tc = static_cast<int>(r % tail_n);
  r /= tail_n;
  const int head = static_cast<int>(r % a.kv_heads);
  r /= a.kv_heads;
  const int layer = static_cast<int>(r % a.n_layers);
  const int b = static_cast<int>(r / a.n_layers);
  const int j = lane & 15, kb = lane >> 4;
  const int rb = j >> 2;  // row block of D
  const int quad = tail_qpc == 2 ? 2 * tc + (rb >> 1) : tc;
  const int oi = min(tail_qpc == 2 ? (rb & 1) : rb, tail_r - 1);
  const int g = min(4 * quad + (j & 3), a.qpk - 1);
  const int64_t row = (static_cast<int64_t>(layer) * a.kv_heads + head) * a.qpk + g;
  const int o = 16 + oi;
  u32x4 hi, lo;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const float v0 = offset_weight(a, b, layer, row, o, m.n_offsets, 32 * st + 8 * kb + 2 * w);
    const float v1 = offset_weight(a, b, layer, row, o, m.n_offsets, 32 * st + 8 * kb + 2 * w + 1);
    const uint32_t h = E::pack(v0, v1);
    hi[w] = h;
    lo[w] = E::pack(v0 - E::lo(h), v1 - E::hi(h));
  }
  const int64_t chunk = ((static_cast<int64_t>(b) * a.n_layers + layer) * a.kv_heads + head) * tail_n + tc;
  u32x4* dst = m.frags + tail_base + (chunk * m.nr + st) * 128 + lane;
  dst[0] = hi;
  dst[64] = lo;
}

// Keys of pages the block table does not resolve read as zeros from here
// (the furthest load reads 16 bytes at element 32 * (NK - 1) + 24).
__device__ __attribute__((aligned(16))) uint32_t kZeroKeys[8 * 16];

// IEEE 754-2019 maximum: NaN if either input is NaN, as torch.maximum
// (one v_maximum3_f32 on gfx950).
__device__ __forceinline__ float max_prop(float a, float b) { return __builtin_elementwise_maximum(a, b); }

// bf16 fragments need no per-column scale.  One workgroup per column
// (sequence, layer, KV head, query head g): its threads first fold the
// weights of every (offset, frequency) with loads along the frequencies into
// an LDS table [offset][rotary dim] (the same expressions as offset_weight),
// then each (chunk and step, operand lane) reads its eight weights from the
// table and writes its hi and lo words.  The table holds n_offsets rows of
// 2F + 4 floats (the padding spreads a lane group's rows over the LDS banks),
// sized by the launch so that small tables leave room for many workgroups.
__host__ __device__ __forceinline__ int fold_table_stride(int freq) { return 2 * freq + 4; }
__global__ __launch_bounds__(256) void fold_offsets_bf16_kernel(OffsetFoldArgs m) {
  typedef MfmaElem<false> E;
  const FoldArgs& a = m.f;
  extern __shared__ __attribute__((aligned(16))) float table[];  // [n_offsets][2F + 4]
  const int kFoldStride = fold_table_stride(a.freq);
  const int64_t col = blockIdx.x;
  const int g = static_cast<int>(col % a.qpk);
  int64_t r = col / a.qpk;
  const int head = static_cast<int>(r % a.kv_heads);
  r /= a.kv_heads;
  const int layer = static_cast<int>(r % a.n_layers);
  const int b = static_cast<int>(r / a.n_layers);
  const int64_t row = (static_cast<int64_t>(layer) * a.kv_heads + head) * a.qpk + g;
  const int F = a.freq;
  for (int i = threadIdx.x; i < m.n_offsets * F; i += blockDim.x) {
    const int o = i / F, f = i - o * F;
    const int64_t ph = b * a.phase_seq_stride + (static_cast<int64_t>(layer) * m.n_offsets + o) * F + f;
    const int64_t q = row * F + f;
    const float qr = a.q_real[q], qi = a.q_imag[q], sc = a.scale[q];
    const float c = a.phase_cos[ph], sn = a.phase_sin[ph];
    float* t = table + o * kFoldStride;
    t[a.interleaved ? 2 * f : f] = sc * (qr * c - qi * sn);
    t[a.interleaved ? 2 * f + 1 : F + f] = sc * (qi * c + qr * sn);
  }
  __syncthreads();
  const int n_pos = m.nch * m.nr;
  u32x4* dst = m.frags + col * n_pos * 2 * 64;
  for (int idx = threadIdx.x; idx < n_pos * 64; idx += blockDim.x) {
    const int lane = idx & 63, p = idx >> 6;
    const int j = lane & 15, kb = lane >> 4;
    const int c = p / m.nr, st = p - c * m.nr;
    const int o = min(16 * c + j, m.n_offsets - 1);
    const float* src = table + o * kFoldStride + 32 * st + 8 * kb;
    u32x4 hi, lo;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float v0 = src[2 * w], v1 = src[2 * w + 1];
      const uint32_t h = E::pack(v0, v1);
      hi[w] = h;
      lo[w] = E::pack(v0 - E::lo(h), v1 - E::hi(h));
    }
    dst[(2 * p) * 64 + lane] = hi;
    dst[(2 * p + 1) * 64 + lane] = lo;
  }
  if (threadIdx.x == 0) m.inv_scale[col] = 1.0f;
}

struct MaxGeometry {
  int gpg;     // query heads per workgroup
  int groups;  // query-head groups per KV head
  int nch;     // 16-offset chunks per query head
  int work;    // (span set, KV head) items
  // Shared tail chunks (16 < offsets <= 20, bf16): offsets 16.. of the query
  // heads in quads, tail_qpc quads per chunk, tail_r rows each; tail_n chunks
  // per KV head, at tail_base (16-byte words) in the fragment region.
  int tail_r, tail_qpc, tail_n;
  int64_t tail_base;
};

// One tile per fragment pass at three waves per SIMD, or two tiles per pass
// at two: the first keeps more key loads in flight, the second halves the
// fragment reads per product.
template <int NK, bool ONE_TILE>
struct MaxTiling {
  static constexpr int T = ONE_TILE || NK >= 8 ? 1 : 2;
  static constexpr int kWavesPerSimd = ONE_TILE ? 3 : 1;  // 1: no request
};

template <int NK, int NF, int NCH, bool F16, bool IL, bool ONE_TILE>
__global__ __launch_bounds__(kScoreThreads)
__attribute__((amdgpu_waves_per_eu(MaxTiling<NK, ONE_TILE>::kWavesPerSimd))) void score_max_kernel(
    ScoreArgs a, MaxGeometry geo, int qpk, const u32x4* __restrict__ rest_frags, const float* __restrict__ rest_scale,
    const u32x4* __restrict__ off_frags, const float* __restrict__ off_scale) {
  typedef MfmaElem<F16> E;
  typedef typename E::vec vec_t;
  constexpr int NR = 2 * NF;   // rotary K steps of 32 dims
  constexpr int NP = NK - NR;  // pass K steps
  constexpr int kNP = NP > 0 ? NP : 1;
  constexpr int kStreams = kScoreThreads / 64;
  constexpr int kQuads = kMfmaMaxQpk / 4;  // quads of query heads in a group
  extern __shared__ u32x4 lds_frag[];      // [gpg][NCH][NR][hi/lo][64], then the tail chunks

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
  const int r = lane & 15;   // token of the tile (B column / D column)
  const int kb = lane >> 4;  // K block of the operands, row block of D
  const int64_t col0 = ((static_cast<int64_t>(b) * a.n_layers + layer) * a.kv_heads + head) * qpk;
  constexpr int kFragPerG = NCH * NR * 2 * 64;
  // Shared tail chunks exist for head_dim >= 128 only (at 64 dims their code
  // would cost the kernel its third wave per SIMD), and not in the one-tile
  // form, which the launcher picks only without them.
  constexpr bool kTail = NCH == 1 && !F16 && NK >= 4 && !ONE_TILE;

  // Stage this group's per-offset fragments.
  {
    const u32x4* src = off_frags + (col0 + g0) * kFragPerG;
    const int count = gcnt * kFragPerG;
#pragma unroll 4
    for (int i = threadIdx.x; i < count; i += kScoreThreads) lds_frag[i] = src[i];
    if constexpr (kTail) if (geo.tail_n > 0) {  // tail chunks after the heads' chunks (one group holds every head)
      const int tcount = geo.tail_n * NR * 128;
      const u32x4* tsrc = off_frags + geo.tail_base + (col0 / qpk) * tcount;
      for (int i = threadIdx.x; i < tcount; i += kScoreThreads) lds_frag[count + i] = tsrc[i];
    }
  }

  // Magnitude and pass fragments (packed [frag][kb][g < qpk], rotary weights
  // zero) as A operands.  Row r takes local query head 4*(r%4) + r/4, so D row
  // 4*kb + i holds local head 4*i + kb: the head that the reduction below
  // leaves in row block kb of quad i.
  constexpr int kFrags = 2 * NK + 2 * NF;
  const int packed = 4 * qpk;
  const int r_head = 4 * (r & 3) + (r >> 2);
  const bool live_row = r_head < gcnt;
  const u32x4* fp = rest_frags + (((static_cast<int64_t>(b) * a.n_layers + layer) * a.kv_heads + head) * kFrags) * packed +
                    kb * qpk + (live_row ? g0 + r_head : 0);
  auto frag_word = [&](int f) {
    const u32x4 v = fp[f * packed];
    return __builtin_bit_cast(vec_t, live_row ? v : u32x4{0, 0, 0, 0});
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

  // Score stage: one row per query head of the group and a spare row that
  // takes the stores of lanes without a head in the group.  In quad q this
  // lane's output is local head 4*q + kb (fp16: with its column scales).
  __shared__ __attribute__((aligned(16))) float stage[(kMfmaMaxQpk + 1) * kStageStride];
  float r_scale[kQuads], o_scale[kQuads];
  float* stage_rows[kQuads];
#pragma unroll
  for (int q = 0; q < kQuads; ++q) {
    const int lh = 4 * q + kb;
    const bool writes = lh < gcnt;
    r_scale[q] = F16 && writes ? rest_scale[col0 + g0 + lh] : 1.0f;
    o_scale[q] = F16 && writes ? off_scale[col0 + g0 + lh] : 1.0f;
    stage_rows[q] = stage + (writes ? lh : kMfmaMaxQpk) * kStageStride + r;
  }

  KVC_GLOBAL const uint16_t* kbase = gptr_from_int<const uint16_t>(a.k_layer_ptrs[layer]);
  const int64_t* bt = a.block_ids + a.block_offsets[b];
  const int64_t n_blocks = a.block_offsets[b + 1] - a.block_offsets[b];
  const int64_t row_elems = static_cast<int64_t>(a.kv_heads) * a.head_dim;
  const int64_t lane_off = static_cast<int64_t>(head) * a.head_dim + 8 * kb;
  const int64_t tok_base = a.token_offsets[b];
  float* raw_out = a.raw + layer * a.raw_layer_stride;
  __syncthreads();  // fragments staged

  // Magnitude + pass term of a tile: D[4*kb + i][r] = local query head 4*i + kb, token r.
  auto rest_tile = [&](const u32x4 (&ka)[NK]) {
    f32x4 acc0 = {0.0f, 0.0f, 0.0f, 0.0f};
    f32x4 acc1 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < NP; ++j) {
      const vec_t kv = __builtin_bit_cast(vec_t, ka[NR + j]);
      if (j & 1) {
        acc1 = E::mfma(p_hi[j], kv, acc1);
        acc1 = E::mfma(p_lo[j], kv, acc1);
      } else {
        acc0 = E::mfma(p_hi[j], kv, acc0);
        acc0 = E::mfma(p_lo[j], kv, acc0);
      }
    }
#pragma unroll
    for (int q = 0; q < NF; ++q) {
      vec_t khi, klo;
      magnitude_operands<F16, IL, NK, NF>(ka, q, &khi, &klo);
      acc0 = E::mfma(m_hi[q], khi, acc0);
      acc1 = E::mfma(m_lo[q], khi, acc1);
      acc0 = E::mfma(m_hi[q], klo, acc0);
    }
    return acc0 + acc1;
  };

  // Keys of a 16-token tile of the span starting at token st0.  Tiles past the
  // span re-read its last tile and rows past the sequence read whatever their
  // page holds: a token is a column of every product here, so those rows only
  // reach scores that are never stored.  Unresolved pages read as zeros.
  auto load_tile = [&](const SpanPages& pg, int st0, int st1, int mt, u32x4 (&ka)[NK]) {
    const int smt = (st1 - st0 + 15) / 16;
    const int mt_read = mt < smt ? mt : smt - 1;
    const int rel = mt_read * 16 + r;
    const int t = st0 + rel;
    bool page_ok = false;
    KVC_GLOBAL const uint16_t* pbase = pg.page(rel, &page_ok);
    KVC_GLOBAL const uint16_t* row =
        page_ok ? pbase + static_cast<int64_t>(t & (kBlockSize - 1)) * row_elems + lane_off
                : reinterpret_cast<KVC_GLOBAL const uint16_t*>(gptr(kZeroKeys));
#pragma unroll
    for (int j = 0; j < NK; ++j) ka[j] = load_k(reinterpret_cast<KVC_GLOBAL const u32x4*>(row + 32 * j));
  };

  // Wave w scores tiles w, w+4, w+8, w+12 of every span in groups of T tiles
  // (T = 2: each fragment read feeds two tiles; T = 1 for head_dim 256,
  // whose key registers would otherwise leave one wave per SIMD, and for the
  // three-waves-per-SIMD form).  The keys of the next group, also across a
  // span boundary and the span's epilogue, are in flight while a group is
  // scored.
  constexpr int T = MaxTiling<NK, ONE_TILE>::T;
  constexpr int kGroups = 4 / T;
  static_assert(kScoreTile == 16 * 4 * kStreams, "four tiles per wave cover a span");
  static_assert(kGroups % 2 == 0, "a span's first group lands in buffer 0");
  const int n_sp = min(kMaxSpans, (n - tile_first * kScoreTile + kScoreTile - 1) / kScoreTile);
  const int n_items = gcnt * NCH;  // one item = one 16-offset chunk of one query head
  const bool tail_pair = geo.tail_qpc == 2;
  u32x4 kbuf[2][T][NK];
  SpanPages pages;
  pages.resolve(kbase, bt, n_blocks, a.num_pages, a.page_stride, tile_first * kScoreTile);
  {
    const int st0 = tile_first * kScoreTile;
    const int st1 = min(n, st0 + kScoreTile);
#pragma unroll
    for (int u = 0; u < T; ++u) load_tile(pages, st0, st1, wave + kStreams * u, kbuf[0][u]);
  }
  for (int sp = 0; sp < n_sp; ++sp) {
    const int tile = tile_first + sp;
    const int t0 = tile * kScoreTile;
    const int t1 = min(n, t0 + kScoreTile);
    const int n_mt = (t1 - t0 + 15) / 16;
    const bool more = sp + 1 < n_sp;
    SpanPages next;  // pages past the table resolve as missing; unused after the last span
    next.resolve(kbase, bt, n_blocks, a.num_pages, a.page_stride, t0 + kScoreTile);

    auto score_group = [&](int mt_first, const u32x4 (&kk)[T][NK]) {
      // Fragments of item it (clamped to the last item) from LDS.
      auto load_w = [&](int it, vec_t (&w)[2 * NR]) {
        const u32x4* wl = lds_frag + (min(it, n_items - 1) * NR) * 128 + lane;
#pragma unroll
        for (int st = 0; st < NR; ++st) {
          w[2 * st] = __builtin_bit_cast(vec_t, wl[st * 128]);
          w[2 * st + 1] = __builtin_bit_cast(vec_t, wl[st * 128 + 64]);
        }
      };
      // Products of the 16 rows of one chunk with the T tiles: D[4*kb + i][r]
      // = row 4*kb + i, token r.  T = 2: one chain per tile, hi then lo;
      // T = 1: hi and lo in separate chains, summed at the end.
      auto chunk_products = [&](const vec_t (&w)[2 * NR], f32x4 (&res)[T]) {
        f32x4 acc[T][2];
#pragma unroll
        for (int u = 0; u < T; ++u) acc[u][0] = acc[u][1] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int st = 0; st < NR; ++st) {
#pragma unroll
          for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int u = 0; u < T; ++u) {
              const int chain = T == 1 ? h : 0;
              acc[u][chain] = E::mfma(w[2 * st + h], __builtin_bit_cast(vec_t, kk[u][st]), acc[u][chain]);
            }
          }
        }
#pragma unroll
        for (int u = 0; u < T; ++u) res[u] = T == 1 ? acc[u][0] + acc[u][1] : acc[u][0];
      };
      auto max4 = [](const f32x4& v) { return max_prop(max_prop(v[0], v[1]), max_prop(v[2], v[3])); };

      f32x4 rest[T];
#pragma unroll
      for (int u = 0; u < T; ++u) rest[u] = rest_tile(kk[u]);
      // Fragment registers: two buffers (the next item's fragments are read
      // while this item's products run), or, in the one-tile form, one buffer
      // whose words are replaced by the next item's as their products issue.
      constexpr int kBufs = ONE_TILE ? 1 : 2;
      vec_t wbuf[kBufs][2 * NR];
      load_w(0, wbuf[0]);
      f32x4 tv[T];
      float outv[T][kQuads];
#pragma unroll
      for (int q = 0; q < kQuads; ++q) {
#pragma unroll
        for (int u = 0; u < T; ++u) outv[u][q] = 0.0f;
        if (4 * q >= gcnt) continue;  // the same for every lane
        // P[u][j]: maximum over the offsets in this lane's row block (D rows
        // 4*kb .. 4*kb + 3 of each chunk) for local head 4*q + j, tile u.
        float P[T][4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
#pragma unroll
          for (int c = 0; c < NCH; ++c) {
            const int it = (4 * q + j) * NCH + c;
            if (4 * q + j < gcnt) {
              f32x4 res[T];
              if constexpr (ONE_TILE) {
                const u32x4* wl = lds_frag + (min(it + 1, n_items - 1) * NR) * 128 + lane;
                f32x4 acc[2] = {f32x4{0.0f, 0.0f, 0.0f, 0.0f}, f32x4{0.0f, 0.0f, 0.0f, 0.0f}};
#pragma unroll
                for (int st = 0; st < NR; ++st) {
#pragma unroll
                  for (int h = 0; h < 2; ++h) {
                    acc[h] = E::mfma(wbuf[0][2 * st + h], __builtin_bit_cast(vec_t, kk[0][st]), acc[h]);
                    wbuf[0][2 * st + h] = __builtin_bit_cast(vec_t, wl[st * 128 + h * 64]);
                  }
                }
                res[0] = acc[0] + acc[1];
              } else {
                load_w(it + 1, wbuf[(it + 1) & 1]);
                chunk_products(wbuf[it & 1], res);
              }
#pragma unroll
              for (int u = 0; u < T; ++u) {
                const float m = max4(res[u]);
                P[u][j] = c == 0 ? m : max_prop(P[u][j], m);
              }
            } else {
#pragma unroll
              for (int u = 0; u < T; ++u) P[u][j] = -INFINITY;
            }
          }
        }
        if constexpr (kTail) if (geo.tail_n > 0) {
          // Tail rows of head 4*q + j are element j of row blocks 2*(q%2) and
          // 2*(q%2) + 1 (two quads a chunk) or of every row block (one).
          if (q == 0 || !tail_pair) {
            vec_t w[2 * NR];
            const u32x4* wl = lds_frag + (n_items + (tail_pair ? 0 : q)) * NR * 128 + lane;
#pragma unroll
            for (int st = 0; st < NR; ++st) {
              w[2 * st] = __builtin_bit_cast(vec_t, wl[st * 128]);
              w[2 * st + 1] = __builtin_bit_cast(vec_t, wl[st * 128 + 64]);
            }
            chunk_products(w, tv);
          }
          const bool take = !tail_pair || (kb >> 1) == (q & 1);
#pragma unroll
          for (int u = 0; u < T; ++u)
#pragma unroll
            for (int j = 0; j < 4; ++j) P[u][j] = max_prop(P[u][j], take ? tv[u][j] : -INFINITY);
        }
        // Maximum over the four row blocks, scattered so that row block kb
        // ends with head 4*q + kb.  v_permlane32_swap(x, y) returns the lower
        // half of x then of y (lanes l and l + 32 of x in lower lane l, of y
        // in upper lane l + 32) and the upper halves; v_permlane16_swap does
        // the same for rows 0/1 and 2/3 of each half.  The maximum of each
        // pair is therefore a maximum over two row blocks of one head.
#pragma unroll
        for (int u = 0; u < T; ++u) {
          const auto s02 = __builtin_amdgcn_permlane32_swap(__float_as_uint(P[u][0]), __float_as_uint(P[u][2]), false, false);
          const float x02 = max_prop(__uint_as_float(s02[0]), __uint_as_float(s02[1]));
          const auto s13 = __builtin_amdgcn_permlane32_swap(__float_as_uint(P[u][1]), __float_as_uint(P[u][3]), false, false);
          const float x13 = max_prop(__uint_as_float(s13[0]), __uint_as_float(s13[1]));
          const auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(x02), __float_as_uint(x13), false, false);
          outv[u][q] = max_prop(__uint_as_float(s[0]), __uint_as_float(s[1]));
        }
      }
      // Column 16*mt + r of the lane's head rows (columns past the span are
      // never read back).
#pragma unroll
      for (int u = 0; u < T; ++u) {
        const int mt = mt_first + kStreams * u;
#pragma unroll
        for (int q = 0; q < kQuads; ++q)
          stage_rows[q][mt * 16] =
              F16 ? outv[u][q] * o_scale[q] + rest[u][q] * r_scale[q] : outv[u][q] + rest[u][q];
      }
    };

#pragma unroll
    for (int q = 0; q < kGroups; ++q) {
      const int cur = q & 1;
      if (q + 1 < kGroups) {
#pragma unroll
        for (int u = 0; u < T; ++u) load_tile(pages, t0, t1, wave + kStreams * ((q + 1) * T + u), kbuf[cur ^ 1][u]);
      } else if (more) {
        const int nt0 = t0 + kScoreTile;
        const int nt1 = min(n, nt0 + kScoreTile);
#pragma unroll
        for (int u = 0; u < T; ++u) load_tile(next, nt0, nt1, wave + kStreams * u, kbuf[cur ^ 1][u]);
      }
      const int mt_first = wave + kStreams * q * T;
      if (mt_first < n_mt) score_group(mt_first, kbuf[cur]);
    }

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
    // Per-head float64 sums of the span's scores for kvc_head_stats: wave w
    // takes rows w, w+4, ...; lane l sums tokens l, l+64, l+128, l+192.
    for (int row = wave; row < gcnt; row += kStreams) {
      double s0 = 0.0, s1 = 0.0;
#pragma unroll
      for (int k = 0; k < kScoreTile / 64; ++k) {
        const int c = lane + 64 * k;
        if (c < span) {
          const double dv = static_cast<double>(stage[row * kStageStride + c]);
          s0 += dv;
          s1 = fma(dv, dv, s1);
        }
      }
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) {
        s0 += __shfl_xor(s0, off);
        s1 += __shfl_xor(s1, off);
      }
      if (lane == 0) {
        const int n_heads = a.kv_heads * qpk;
        double* dst = a.partials +
                      (((static_cast<int64_t>(layer) * a.n_seq + b) * a.max_tiles + tile) * n_heads + q_first + row) * 2;
        dst[0] = s0;
        dst[1] = s1;
      }
    }
    __syncthreads();  // stage and red are reused by the next span
    pages = next;
  }
}

// ------------------------------------------------------- vector-ALU path --

// Shapes the matrix-core scorer does not serve (F not a multiple of 32, or
// head_dim other than 64/128/256): one thread per token of a 256-token span
// for one query head.  The workgroup folds that head's per-offset weights
// (real / imaginary part per frequency, rows past the last offset repeating
// it) and its magnitude and pass weights into LDS, then each thread walks its
// key row in blocks of 8 frequencies (16-byte loads of the real and the
// imaginary parts), accumulating 16*NCH offset sums, the magnitude term and
// the pass term; LDS weight reads are wave-wide broadcasts.
constexpr int kValuMaxLds = 64 * 1024;

template <typename Tag, bool IL, int NCH>
__global__ __launch_bounds__(256) void score_max_valu_kernel(ScoreArgs a, FoldArgs f, int qpk, int n_offsets) {
  constexpr int OO = 16 * NCH;
  extern __shared__ __attribute__((aligned(16))) float lds_w[];  // wre[OO][F], wim[OO][F], wm[F], wp[P]
  const int F = a.freq, P = a.head_dim - a.rotary_dim;
  float* wre = lds_w;
  float* wim = wre + OO * F;
  float* wm = wim + OO * F;
  float* wp = wm + F;
  const int n_heads = a.kv_heads * qpk;
  const int q = blockIdx.z % n_heads;
  const int layer = blockIdx.z / n_heads;
  const int b = blockIdx.y;
  const int tile = blockIdx.x;
  const int n = a.seq_lens[b];
  const int t0 = tile * kScoreTile;
  if (t0 >= n) return;  // whole workgroup
  const int head = q / qpk, g = q - head * qpk;
  const int64_t row = (static_cast<int64_t>(layer) * a.kv_heads + head) * qpk + g;

  for (int i = threadIdx.x; i < OO * F; i += blockDim.x) {
    const int o = min(i / F, n_offsets - 1), fr = i - (i / F) * F;
    const int64_t ph = b * f.phase_seq_stride + (static_cast<int64_t>(layer) * n_offsets + o) * F + fr;
    const int64_t qi_ = row * F + fr;
    const float qr = f.q_real[qi_], qi = f.q_imag[qi_], sc = f.scale[qi_];
    const float c = f.phase_cos[ph], sn = f.phase_sin[ph];
    wre[i] = sc * (qr * c - qi * sn);
    wim[i] = sc * (qi * c + qr * sn);
  }
  for (int i = threadIdx.x; i < F; i += blockDim.x) wm[i] = f.scale[row * F + i] * f.extra[row * F + i];
  for (int i = threadIdx.x; i < P; i += blockDim.x) wp[i] = f.q_pass[row * P + i];
  __syncthreads();

  const int t = t0 + threadIdx.x;
  const bool valid = t < n;
  KVC_GLOBAL const uint16_t* kbase = gptr_from_int<const uint16_t>(a.k_layer_ptrs[layer]);
  const int64_t* bt = a.block_ids + a.block_offsets[b];
  const int64_t n_blocks = a.block_offsets[b + 1] - a.block_offsets[b];
  const int64_t blk = valid ? (t >> kBlockShift) : 0;
  const int64_t page = blk < n_blocks ? bt[blk] : -1;
  const bool page_ok = valid && page >= 0 && page < a.num_pages;
  KVC_GLOBAL const uint16_t* krow =
      kbase + (page_ok ? page : 0) * a.page_stride +
      static_cast<int64_t>(t & (kBlockSize - 1)) * a.kv_heads * a.head_dim + static_cast<int64_t>(head) * a.head_dim;

  float acc[OO];
#pragma unroll
  for (int o = 0; o < OO; ++o) acc[o] = 0.0f;
  float mag = 0.0f, pass = 0.0f;
  typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
  for (int fb = 0; fb < F; fb += 8) {
    u32x4_t va = {0, 0, 0, 0}, vb = {0, 0, 0, 0};
    if (page_ok) {
      va = *reinterpret_cast<KVC_GLOBAL const u32x4_t*>(krow + (IL ? 2 * fb : fb));
      vb = *reinterpret_cast<KVC_GLOBAL const u32x4_t*>(krow + (IL ? 2 * fb + 8 : F + fb));
    }
    float re[8], im[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (IL) {  // (re, im) pairs: va holds frequencies fb..fb+3, vb fb+4..fb+7
        re[j] = Unpack<Tag>::lo(va[j]);
        im[j] = Unpack<Tag>::hi(va[j]);
        re[4 + j] = Unpack<Tag>::lo(vb[j]);
        im[4 + j] = Unpack<Tag>::hi(vb[j]);
      } else {
        re[2 * j] = Unpack<Tag>::lo(va[j]);
        re[2 * j + 1] = Unpack<Tag>::hi(va[j]);
        im[2 * j] = Unpack<Tag>::lo(vb[j]);
        im[2 * j + 1] = Unpack<Tag>::hi(vb[j]);
      }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) mag = fmaf(wm[fb + j], __builtin_amdgcn_sqrtf(fmaf(im[j], im[j], re[j] * re[j])), mag);
#pragma unroll
    for (int o = 0; o < OO; ++o) {
      const float* r_ = wre + o * F + fb;
      const float* i_ = wim + o * F + fb;
      float v = acc[o];
#pragma unroll
      for (int j = 0; j < 8; ++j) v = fmaf(r_[j], re[j], fmaf(i_[j], im[j], v));
      acc[o] = v;
    }
  }
  for (int pb = 0; pb < P; pb += 8) {
    u32x4_t v = {0, 0, 0, 0};
    if (page_ok) v = *reinterpret_cast<KVC_GLOBAL const u32x4_t*>(krow + a.rotary_dim + pb);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      pass = fmaf(wp[pb + 2 * j], Unpack<Tag>::lo(v[j]), pass);
      pass = fmaf(wp[pb + 2 * j + 1], Unpack<Tag>::hi(v[j]), pass);
    }
  }
  float best = acc[0];
#pragma unroll
  for (int o = 1; o < OO; ++o) best = max_prop(best, acc[o]);
  const float score = best + mag + pass;

  double s0 = 0.0, s1 = 0.0;
  if (valid) {
    a.raw[layer * a.raw_layer_stride + (a.token_offsets[b] + t) * a.raw_token_stride + q * a.raw_head_stride] = score;
    s0 = static_cast<double>(score);
    s1 = s0 * s0;
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    s0 += __shfl_xor(s0, off);
    s1 += __shfl_xor(s1, off);
  }
  __shared__ double red[2][4];
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    red[0][wave] = s0;
    red[1][wave] = s1;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    double* dst = a.partials + (((static_cast<int64_t>(layer) * a.n_seq + b) * a.max_tiles + tile) * n_heads + q) * 2;
    dst[0] = red[0][0] + red[0][1] + red[0][2] + red[0][3];
    dst[1] = red[1][0] + red[1][1] + red[1][2] + red[1][3];
  }
}

using ValuMaxKernel = void (*)(ScoreArgs, FoldArgs, int, int);

template <typename Tag, bool IL>
ValuMaxKernel pick_valu_max(int nch) {
  if (nch == 1) return score_max_valu_kernel<Tag, IL, 1>;
  if (nch == 2) return score_max_valu_kernel<Tag, IL, 2>;
  return nullptr;
}

using MaxKernel = void (*)(ScoreArgs, MaxGeometry, int, const u32x4*, const float*, const u32x4*, const float*);

template <int NCH, bool F16, bool IL>
MaxKernel pick_max_chunks(int nk, int nf, bool one_tile) {
  if (one_tile) {  // head_dim 128, one chunk per query head, no tail chunks
    if (NCH != 1 || nk != 4) return nullptr;
    return nf == 1 ? score_max_kernel<4, 1, 1, F16, IL, true> : nf == 2 ? score_max_kernel<4, 2, 1, F16, IL, true> : nullptr;
  }
  switch (nk * 16 + nf) {
    case 2 * 16 + 1: return score_max_kernel<2, 1, NCH, F16, IL, false>;
    case 4 * 16 + 1: return score_max_kernel<4, 1, NCH, F16, IL, false>;
    case 4 * 16 + 2: return score_max_kernel<4, 2, NCH, F16, IL, false>;
    case 8 * 16 + 1: return score_max_kernel<8, 1, NCH, F16, IL, false>;
    case 8 * 16 + 2: return score_max_kernel<8, 2, NCH, F16, IL, false>;
    case 8 * 16 + 4: return score_max_kernel<8, 4, NCH, F16, IL, false>;
    default: return nullptr;
  }
}

template <bool F16, bool IL>
MaxKernel pick_max_typed(int nk, int nf, int nch, bool one_tile) {
  if (nch == 1) return pick_max_chunks<1, F16, IL>(nk, nf, one_tile);
  if (nch == 2) return pick_max_chunks<2, F16, IL>(nk, nf, one_tile);
  return nullptr;
}

}  // namespace

int launch_max_scorer(hipStream_t stream, const ScoreShape& s, int dtype, int n_offsets, const FoldArgs& fa,
                      const ScoreArgs& sa, void* workspace) {
  const int nk = s.head_dim / 32, nf = s.freq / 32, nr = 2 * nf;
  const bool f16 = dtype == KVC_DTYPE_FP16;
  MaxGeometry geo;
  geo.nch = offset_chunks(n_offsets);
  if (geo.nch > 2)
    return fail(KVC_EINVAL, "kvc_score_paged_max: at most 32 offsets (got %d; 2^0 .. 2^30 are 31)", n_offsets);
  int nch = geo.nch;
  geo.tail_r = geo.tail_qpc = geo.tail_n = 0;
  geo.tail_base = 0;
  if (!mfma_scorer_supported(s, dtype, fa.interleaved ? KVC_ROPE_INTERLEAVED : KVC_ROPE_HALF)) {
    const size_t lds = sizeof(float) * (2 * static_cast<size_t>(16 * nch) * s.freq + s.freq + s.pass);
    if (lds > static_cast<size_t>(kValuMaxLds))
      return fail(KVC_EINVAL, "kvc_score_paged_max: %d offsets x %d frequencies exceed the LDS of one workgroup",
                  n_offsets, s.freq);
    const int64_t gz = static_cast<int64_t>(s.n_layers) * s.kv_heads * s.qpk;
    if (gz > 65535) return fail(KVC_EINVAL, "kvc_score_paged_max: too many layers x query heads for one launch");
    ValuMaxKernel vk = f16 ? (fa.interleaved ? pick_valu_max<Fp16Tag, true>(nch) : pick_valu_max<Fp16Tag, false>(nch))
                           : (fa.interleaved ? pick_valu_max<Bf16Tag, true>(nch) : pick_valu_max<Bf16Tag, false>(nch));
    dim3 grid(static_cast<unsigned>(s.max_tiles), static_cast<unsigned>(s.n_seq), static_cast<unsigned>(gz));
    vk<<<grid, 256, lds, stream>>>(sa, fa, s.qpk, n_offsets);
    return launch_status("kvc_score_paged_max");
  }
  // 17 to 20 offsets (bf16): each query head keeps one 16-offset chunk and the
  // remaining 1-4 offsets of its quad of heads share tail chunks (two quads a
  // chunk for 1-2 remaining offsets), when every head of the KV head then fits
  // one workgroup (18 offsets, 5 query heads, 128 dims: 6 chunk passes per
  // tile instead of 10, and keys read once).
  const int64_t cols_total = static_cast<int64_t>(s.n_seq) * s.n_layers * s.kv_heads * s.qpk;
  if (!f16 && nk >= 4 && n_offsets > 16 && n_offsets <= 20) {
    const int r = n_offsets - 16, qpc = r <= 2 ? 2 : 1;
    const int tn = ((s.qpk + 3) / 4 + qpc - 1) / qpc;
    if ((s.qpk + tn) * nr * 2 * kOffsetFragBytes <= kMaxFragLds) {
      geo.nch = nch = 1;
      geo.tail_r = r;
      geo.tail_qpc = qpc;
      geo.tail_n = tn;
      geo.tail_base = cols_total * nr * 128;
    }
  }
  // One tile per pass at three waves per SIMD where that measured faster: 128
  // dims with one chunk per query head and no tail (16 offsets, Qwen2.5-14B
  // shape: 1.03 against 1.13 ms; with a tail chunk it is 9% slower).
  const bool one_tile = nk == 4 && nch == 1 && geo.tail_n == 0;
  MaxKernel kern =
      f16 ? (fa.interleaved ? pick_max_typed<true, true>(nk, nf, nch, one_tile) : pick_max_typed<true, false>(nk, nf, nch, one_tile))
          : (fa.interleaved ? pick_max_typed<false, true>(nk, nf, nch, one_tile)
                            : pick_max_typed<false, false>(nk, nf, nch, one_tile));
  if (!kern) return fail(KVC_EINVAL, "kvc_score_paged_max: no scorer for head_dim %d rotary_dim %d", s.head_dim, s.rotary_dim);
  const int per_g = geo.nch * nr * 2 * kOffsetFragBytes;
  int gpg = kMaxFragLds / per_g;
  if (geo.tail_n > 0) gpg = s.qpk;
  if (gpg < 1)
    return fail(KVC_EINVAL, "kvc_score_paged_max: %d offsets need %d bytes of fragments per query head (limit %d)",
                n_offsets, per_g, kMaxFragLds);
  if (gpg > s.qpk) gpg = s.qpk;
  geo.groups = (s.qpk + gpg - 1) / gpg;
  geo.gpg = (s.qpk + geo.groups - 1) / geo.groups;
  const int64_t items = ceil_div(s.max_tiles, kMaxSpans) * s.kv_heads;
  const int64_t gx = ceil_div(items, 8) * 8 * geo.groups;
  if (gx > 0x7fffffff) return fail(KVC_EINVAL, "kvc_score_paged_max: grid too large");
  // Every fold this call launches, checked before the first of them: the
  // magnitude/pass fold, the per-offset fold (fp16: one wave per column, four
  // per workgroup; bf16: one workgroup per column) and the tail fold.
  // bf16 fold: one workgroup per column, its offset table in LDS (at most 32
  // offsets x 260 floats here: 33 KB).
  const size_t fold_lds = static_cast<size_t>(n_offsets) * fold_table_stride(s.freq) * sizeof(float);
  const int64_t offset_items = f16 ? ceil_div(cols_total, 4) * 256 : cols_total * 256;
  const int64_t tail_items =
      geo.tail_n > 0 ? ceil_div(cols_total / s.qpk * geo.tail_n * nr * 64, 256) * 256 : 0;
  const int64_t fold_items = std::max(mfma_fold_items(s, dtype), std::max(offset_items, tail_items));
  if (fold_items > kMaxDispatchItems)
    return fail(KVC_EINVAL, "kvc_score_paged_max: the weight folds of %lld columns exceed one dispatch",
                static_cast<long long>(cols_total));
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
  if (f16)
    fold_offsets_kernel<true><<<static_cast<unsigned>(offset_items / 256), 256, 0, stream>>>(m);
  else
    fold_offsets_bf16_kernel<<<static_cast<unsigned>(offset_items / 256), 256, fold_lds, stream>>>(m);
  if (int rc = launch_status("kvc_score_paged_max(fold)")) return rc;
  if (geo.tail_n > 0) {
    fold_offsets_tail_bf16_kernel<<<static_cast<unsigned>(tail_items / 256), 256, 0, stream>>>(
        m, geo.tail_r, geo.tail_qpc, geo.tail_n, geo.tail_base);
    if (int rc = launch_status("kvc_score_paged_max(tail fold)")) return rc;
  }

  const float* rest_scale =
      reinterpret_cast<const float*>(static_cast<const char*>(workspace) + mfma_fragment_only_bytes(s));
  const size_t lds = static_cast<size_t>(geo.gpg) * per_g + static_cast<size_t>(geo.tail_n) * nr * 2 * kOffsetFragBytes;
  dim3 grid(static_cast<unsigned>(gx), static_cast<unsigned>(s.n_seq), static_cast<unsigned>(s.n_layers));
  kern<<<grid, kScoreThreads, lds, stream>>>(sa, geo, s.qpk, static_cast<const u32x4*>(workspace), rest_scale, m.frags,
                                             m.inv_scale);
  return launch_status("kvc_score_paged_max");
}

}  // namespace kvc
