// Pre-RoPE query statistics for a calibration artifact, on CDNA4.
//
// The calibration generator hooks every full-attention layer's query
// projection and reduces it over tokens (_LayerAccumulator.add,
// pkg/calibration.py:98-131).  With F = rotary_dim/2 frequencies and
// P = head_dim - rotary_dim pass dims, for every query head h:
//   real_sum[h][f] = sum_t q[t][h][f]                           f < F
//   imag_sum[h][f] = sum_t q[t][h][F + f]
//   abs_sum[h][f]  = sum_t sqrt(q[t][h][f]^2 + q[t][h][F + f]^2)
//   pass_sum[h][p] = sum_t q[t][h][rotary_dim + p]               p < P
// Each element is widened to float32 and the magnitude is formed as the
// reference forms it (two float32 squares, one add, a correctly rounded
// square root; no fused multiply-add), so every per-token term is the
// reference's; the sums are float64.
//
// A unit is one frequency (its real and imaginary dim) or one pass dim of one
// head.  A lane owns V consecutive units (V = 4 where the shape and the
// addresses allow vector loads, else 1).  The accumulation grid is (blocks of
// 64 lanes) x (token splits): a workgroup of 4 waves covers 64*V units over
// one split's tokens, wave w summing the split's tokens t = w (mod 4) with 8
// tokens' loads in flight; the four wave partials are combined in wave order
// in LDS and added into the caller's state at [split][unit][3].  Every state
// entry has one owner per launch, so calls add up in call order, and the
// finish kernel sums a unit's splits in split order: repeated runs give
// identical sums.  Accumulation reads the projections once (bound: HBM, 2-4
// bytes per element); the state is 128 splits x units x 24 bytes.

#include "kvc_common.h"

namespace kvc {
namespace {

constexpr int kQsWaves = 4;
constexpr int kQsThreads = kQsWaves * 64;
constexpr int kQsUnroll = 8;
constexpr int kQsSplits = 128;         // state rows
constexpr int kQsMinSplitTokens = 32;  // tokens per split, at least

struct QStatsArgs {
  const void* q;
  int64_t n_tokens, token_stride, split_tokens;
  int heads, head_dim, freq, pass;
  double* state;  // [kQsSplits][units][3]
};

inline int64_t qstats_units(int heads, int head_dim, int rotary_dim) {
  return static_cast<int64_t>(heads) * (rotary_dim / 2 + head_dim - rotary_dim);
}

template <typename T>
__device__ __forceinline__ float widen(T v);
template <>
__device__ __forceinline__ float widen<uint16_t>(uint16_t v) {  // bf16 bits
  return __uint_as_float(static_cast<uint32_t>(v) << 16);
}
template <>
__device__ __forceinline__ float widen<_Float16>(_Float16 v) {
  return static_cast<float>(v);
}
template <>
__device__ __forceinline__ float widen<float>(float v) {
  return v;
}

// V consecutive elements widened to float32, read with one load of
// V*sizeof(T) bytes (aligned by the host).
template <typename T, int V>
__device__ __forceinline__ void load_widen(KVC_GLOBAL const T* p, float (&out)[V]) {
  if constexpr (V == 1) {
    out[0] = widen<T>(*p);
  } else {
    typedef T vec_t __attribute__((ext_vector_type(V)));
    const vec_t x = *reinterpret_cast<KVC_GLOBAL const vec_t*>(p);
#pragma unroll
    for (int e = 0; e < V; ++e) out[e] = widen<T>(x[e]);
  }
}

template <typename T, int V>
__global__ __launch_bounds__(kQsThreads) void qstats_accumulate_kernel(QStatsArgs a) {
  __shared__ double red[kQsWaves][3 * V][64];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int fg = a.freq / V, pg = a.pass / V;  // unit groups per head
  const int64_t groups = static_cast<int64_t>(a.heads) * (fg + pg);
  const int64_t group = static_cast<int64_t>(blockIdx.x) * 64 + lane;
  const bool live = group < groups;
  const int h = live ? static_cast<int>(group / (fg + pg)) : 0;
  const int c = live ? static_cast<int>(group - static_cast<int64_t>(h) * (fg + pg)) : 0;
  const bool pair = c < fg;
  // Row offsets: real dims f0.., imaginary F+f0.. for frequencies; R+p0.. for pass dims.
  const int64_t d0 = static_cast<int64_t>(h) * a.head_dim + (pair ? c * V : 2 * a.freq + (c - fg) * V);
  const int64_t d1 = pair ? d0 + a.freq : d0;
  KVC_GLOBAL const T* q = gptr(static_cast<const T*>(a.q));
  const int64_t begin = static_cast<int64_t>(blockIdx.y) * a.split_tokens;
  const int64_t end = min(a.n_tokens, begin + a.split_tokens);

  double s_re[V], s_im[V], s_abs[V];
#pragma unroll
  for (int e = 0; e < V; ++e) s_re[e] = s_im[e] = s_abs[e] = 0.0;
  if (live) {
    for (int64_t t0 = begin + wave; t0 < end; t0 += static_cast<int64_t>(kQsWaves) * kQsUnroll) {
      float re[kQsUnroll][V], im[kQsUnroll][V];
#pragma unroll
      for (int u = 0; u < kQsUnroll; ++u) {
        const int64_t t = t0 + static_cast<int64_t>(u) * kQsWaves;
        const int64_t row = (t < end ? t : t0) * a.token_stride;  // in range; surplus ignored
        load_widen<T, V>(q + row + d0, re[u]);
        load_widen<T, V>(q + row + d1, im[u]);
      }
#pragma unroll
      for (int u = 0; u < kQsUnroll; ++u) {
        if (t0 + static_cast<int64_t>(u) * kQsWaves < end) {
#pragma unroll
          for (int e = 0; e < V; ++e) {
            const float x = re[u][e], y = im[u][e];
            s_re[e] += static_cast<double>(x);
            s_im[e] += static_cast<double>(y);
            s_abs[e] += static_cast<double>(__fsqrt_rn(__fadd_rn(__fmul_rn(x, x), __fmul_rn(y, y))));
          }
        }
      }
    }
  }
#pragma unroll
  for (int e = 0; e < V; ++e) {
    red[wave][3 * e][lane] = s_re[e];
    red[wave][3 * e + 1][lane] = s_im[e];
    red[wave][3 * e + 2][lane] = s_abs[e];
  }
  __syncthreads();
  if (wave != 0 || !live) return;
  const int64_t units = static_cast<int64_t>(a.heads) * (a.freq + a.pass);
  // Unit index of element e: frequencies h*(F+P) + f, pass dims h*(F+P) + F + p.
  const int64_t unit0 = static_cast<int64_t>(h) * (a.freq + a.pass) + (pair ? c * V : a.freq + (c - fg) * V);
  double* st = a.state + (static_cast<int64_t>(blockIdx.y) * units + unit0) * 3;
#pragma unroll
  for (int k = 0; k < 3 * V; ++k) {
    double r = 0.0;
#pragma unroll
    for (int w = 0; w < kQsWaves; ++w) r += red[w][k][lane];
    st[k] += r;  // element e, statistic k%3 at unit0 + e: [e][3] is contiguous
  }
}

__global__ void qstats_finish_kernel(const double* __restrict__ state, int64_t units, int heads, int freq, int pass,
                                     double* __restrict__ real_sum, double* __restrict__ imag_sum,
                                     double* __restrict__ abs_sum, double* __restrict__ pass_sum) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;  // unit*3 + statistic
  if (idx >= units * 3) return;
  // Splits in order, 16 loads in flight at a time.
  double sum = 0.0;
  for (int s0 = 0; s0 < kQsSplits; s0 += 16) {
    double r[16];
#pragma unroll
    for (int s = 0; s < 16; ++s) r[s] = state[static_cast<int64_t>(s0 + s) * units * 3 + idx];
#pragma unroll
    for (int s = 0; s < 16; ++s) sum += r[s];
  }
  const int64_t unit = idx / 3;
  const int k = static_cast<int>(idx - unit * 3);
  const int h = static_cast<int>(unit / (freq + pass));
  const int c = static_cast<int>(unit - static_cast<int64_t>(h) * (freq + pass));
  if (c < freq) {
    double* out = k == 0 ? real_sum : (k == 1 ? imag_sum : abs_sum);
    out[static_cast<int64_t>(h) * freq + c] = sum;
  } else if (k == 0) {
    pass_sum[static_cast<int64_t>(h) * pass + (c - freq)] = sum;
  }
}

bool shape_ok(int heads, int head_dim, int rotary_dim) {
  return heads > 0 && head_dim > 0 && rotary_dim > 0 && rotary_dim <= head_dim && rotary_dim % 2 == 0;
}

}  // namespace
}  // namespace kvc

using namespace kvc;

extern "C" size_t kvc_qstats_state_bytes(int heads, int head_dim, int rotary_dim) {
  if (!shape_ok(heads, head_dim, rotary_dim)) return 0;
  return static_cast<size_t>(kQsSplits) * qstats_units(heads, head_dim, rotary_dim) * 3 * sizeof(double);
}

extern "C" int kvc_qstats_accumulate(kvc_stream_t stream, int dtype, const void* q, int64_t n_tokens,
                                     int64_t token_stride, int heads, int head_dim, int rotary_dim, void* state,
                                     size_t state_bytes) {
  if (dtype != KVC_DTYPE_BF16 && dtype != KVC_DTYPE_FP16 && dtype != KVC_DTYPE_FP32)
    return fail(KVC_EINVAL, "kvc_qstats_accumulate: unknown dtype %d", dtype);
  if (heads <= 0 || head_dim <= 0 || n_tokens < 0) return fail(KVC_EINVAL, "kvc_qstats_accumulate: bad sizes");
  if (!shape_ok(heads, head_dim, rotary_dim))
    return fail(KVC_EINVAL, "kvc_qstats_accumulate: rotary_dim must be positive, even and <= head_dim");
  if (token_stride < static_cast<int64_t>(heads) * head_dim)
    return fail(KVC_EINVAL, "kvc_qstats_accumulate: token_stride smaller than a token's row");
  const size_t need = kvc_qstats_state_bytes(heads, head_dim, rotary_dim);
  if (!state || state_bytes < need)
    return fail(KVC_EINVAL, "kvc_qstats_accumulate: state of %zu bytes needed", need);
  if (n_tokens == 0) return 0;
  if (!q) return fail(KVC_EINVAL, "kvc_qstats_accumulate: null input");
  QStatsArgs a;
  a.q = q;
  a.n_tokens = n_tokens;
  a.token_stride = token_stride;
  a.heads = heads;
  a.head_dim = head_dim;
  a.freq = rotary_dim / 2;
  a.pass = head_dim - rotary_dim;
  a.state = static_cast<double*>(state);
  int64_t splits = ceil_div(n_tokens, kQsMinSplitTokens);
  if (splits > kQsSplits) splits = kQsSplits;
  a.split_tokens = ceil_div(n_tokens, splits);
  splits = ceil_div(n_tokens, a.split_tokens);

  const int esize = dtype == KVC_DTYPE_FP32 ? 4 : 2;
  // Four-wide loads need every vector start aligned: frequency and pass
  // blocks, the head dim, the token stride and the base address.
  const bool wide = a.freq % 4 == 0 && a.pass % 4 == 0 && token_stride % 4 == 0 &&
                    reinterpret_cast<uintptr_t>(q) % (4 * esize) == 0;
  const int v = wide ? 4 : 1;
  const int64_t groups = static_cast<int64_t>(heads) * (a.freq / v + a.pass / v);
  const int64_t blocks = ceil_div(groups, 64);
  if (blocks > 0x7fffffff) return fail(KVC_EINVAL, "kvc_qstats_accumulate: too many heads");
  const dim3 grid(static_cast<unsigned>(blocks), static_cast<unsigned>(splits));
  hipStream_t st = as_stream(stream);
  switch (dtype * 2 + (wide ? 1 : 0)) {
    case KVC_DTYPE_BF16 * 2 + 1: qstats_accumulate_kernel<uint16_t, 4><<<grid, kQsThreads, 0, st>>>(a); break;
    case KVC_DTYPE_BF16 * 2: qstats_accumulate_kernel<uint16_t, 1><<<grid, kQsThreads, 0, st>>>(a); break;
    case KVC_DTYPE_FP16 * 2 + 1: qstats_accumulate_kernel<_Float16, 4><<<grid, kQsThreads, 0, st>>>(a); break;
    case KVC_DTYPE_FP16 * 2: qstats_accumulate_kernel<_Float16, 1><<<grid, kQsThreads, 0, st>>>(a); break;
    case KVC_DTYPE_FP32 * 2 + 1: qstats_accumulate_kernel<float, 4><<<grid, kQsThreads, 0, st>>>(a); break;
    default: qstats_accumulate_kernel<float, 1><<<grid, kQsThreads, 0, st>>>(a); break;
  }
  return launch_status("kvc_qstats_accumulate");
}

extern "C" int kvc_qstats_finish(kvc_stream_t stream, int heads, int head_dim, int rotary_dim, const void* state,
                                 double* real_sum, double* imag_sum, double* abs_sum, double* pass_sum) {
  if (!shape_ok(heads, head_dim, rotary_dim))
    return fail(KVC_EINVAL, "kvc_qstats_finish: heads, head_dim and an even rotary_dim <= head_dim are required");
  const int pass = head_dim - rotary_dim;
  if (!state || !real_sum || !imag_sum || !abs_sum || (pass > 0 && !pass_sum))
    return fail(KVC_EINVAL, "kvc_qstats_finish: null pointer");
  const int64_t units = qstats_units(heads, head_dim, rotary_dim);
  qstats_finish_kernel<<<static_cast<unsigned>(ceil_div(units * 3, 256)), 256, 0, as_stream(stream)>>>(
      static_cast<const double*>(state), units, heads, rotary_dim / 2, pass, real_sum, imag_sum, abs_sum, pass_sum);
  return launch_status("kvc_qstats_finish");
}
