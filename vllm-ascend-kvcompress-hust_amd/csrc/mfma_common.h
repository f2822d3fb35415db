// Matrix-core helpers shared by the mean scorer (score_mfma.hip) and the
// max-over-offsets scorer (score_max.hip).
#pragma once

#include "score_internal.h"

namespace kvc {

constexpr int kMfmaMaxQpk = 8;                // make_shape admits qpk <= 8
constexpr int kStageStride = kScoreTile + 4;  // floats per staged query-head row

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Two floats -> packed bf16 pair, round to nearest even (one v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
}
// Two floats -> packed fp16 pair, round to nearest even (one v_cvt_pk_f16_f32).
__device__ __forceinline__ uint32_t pack_f16(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, f16x2));
}

// The 16-bit element type of a cache: A/B operand vector, the MFMA, the
// unpacking and hi/lo packing of |k|.
template <bool F16>
struct MfmaElem;
template <>
struct MfmaElem<false> {
  typedef bf16x8 vec;
  static constexpr float kMagScale = 1.0f;
  __device__ __forceinline__ static f32x4 mfma(vec a, vec b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  __device__ __forceinline__ static float lo(uint32_t w) { return bf16_lo(w); }
  __device__ __forceinline__ static float hi(uint32_t w) { return bf16_hi(w); }
  __device__ __forceinline__ static uint32_t pack(float a, float b) { return pack_bf16(a, b); }
};
template <>
struct MfmaElem<true> {
  typedef f16x8 vec;
  static constexpr float kMagScale = 0.25f;  // |k| of fp16 keys reaches 2^16.5
  __device__ __forceinline__ static f32x4 mfma(vec a, vec b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  __device__ __forceinline__ static float lo(uint32_t w) { return fp16_lo(w); }
  __device__ __forceinline__ static float hi(uint32_t w) { return fp16_hi(w); }
  __device__ __forceinline__ static uint32_t pack(float a, float b) { return pack_f16(a, b); }
};

// K is read once per scoring layer, with plain loads: non-temporal ones
// (meant to keep K from evicting the weight fragments in L2) measured 0.85 ms
// against 0.72 ms on the Qwen2.5-14B shape.
__device__ __forceinline__ u32x4 load_k(KVC_GLOBAL const u32x4* p) {
  return *p;
}

// Round-to-nearest-even float32 -> bf16 bits (finite inputs).
__device__ __forceinline__ uint32_t bf16_bits(float x) {
  const uint32_t u = __float_as_uint(x);
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}
__device__ __forceinline__ float bf16_value(uint32_t bits) { return __uint_as_float(bits << 16); }

// |k| of the eight frequencies of magnitude K step q held by this lane, as
// hi/lo 16-bit A operands (hi + lo = |k| * kMagScale to ~2^-16).  Two
// frequencies per output word: half style pairs word w of linear steps q
// (real parts) and q + NF (imaginary parts); interleaved takes words 2w, 2w+1
// of step 2q (w < 2) or 2q + 1, each word one (real, imaginary) pair.
template <bool F16, bool IL, int NK, int NF>
__device__ __forceinline__ void magnitude_operands(const u32x4 (&ka)[NK], int q, typename MfmaElem<F16>::vec* khi,
                                                   typename MfmaElem<F16>::vec* klo) {
  typedef MfmaElem<F16> E;
  typedef typename E::vec vec_t;
  u32x4 hi, lo;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    uint32_t re_w, im_w;
    if (IL) {
      const uint32_t w0 = ka[2 * q + (w >> 1)][(2 * w) & 3], w1 = ka[2 * q + (w >> 1)][(2 * w + 1) & 3];
      // (re0, re1) = (lo of w0, lo of w1), (im0, im1) = (hi of w0, hi of w1)
      re_w = (w0 & 0xffffu) | (w1 << 16);
      im_w = (w0 >> 16) | (w1 & 0xffff0000u);
    } else {
      re_w = ka[q][w];
      im_w = ka[q + NF][w];
    }
    const float re0 = E::lo(re_w), re1 = E::hi(re_w);
    const float im0 = E::lo(im_w), im1 = E::hi(im_w);
    const float m0 = __builtin_amdgcn_sqrtf(fmaf(im0, im0, re0 * re0)) * E::kMagScale;
    const float m1 = __builtin_amdgcn_sqrtf(fmaf(im1, im1, re1 * re1)) * E::kMagScale;
    const uint32_t hw = E::pack(m0, m1);
    hi[w] = hw;
    lo[w] = E::pack(m0 - E::lo(hw), m1 - E::hi(hw));
  }
  *khi = __builtin_bit_cast(vec_t, hi);
  *klo = __builtin_bit_cast(vec_t, lo);
}

}  // namespace kvc
