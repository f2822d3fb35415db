// Shared device helpers and host-side error reporting for the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kvcompress_mi355x.h"

namespace kvc {

// Token rows per cache page (reference ASCEND_BLOCK_SIZE).
constexpr int kBlockShift = 7;
constexpr int kBlockSize = 1 << kBlockShift;

// Host: record a message for kvc_last_error() and return `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Host: translate a launch status into the ABI's return convention.
int launch_status(const char* what);

inline hipStream_t as_stream(kvc_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// ------------------------------------------------------------------ device --

// Global-memory (address space 1) views of device pointers.  Cache base
// addresses arrive as integers in per-layer tables, and a pointer made from
// an integer is generic: its loads and stores compile to flat_* instructions,
// which also count against the scalar-memory wait counter, so the first wait
// for a scalar load (a table entry, a kernel argument) drains every vector
// load in flight.  global_* instructions count only against the vector one.
#define KVC_GLOBAL __attribute__((address_space(1)))
template <typename T>
__device__ __forceinline__ KVC_GLOBAL const T* gptr(const T* p) {
  return (KVC_GLOBAL const T*)p;
}
template <typename T>
__device__ __forceinline__ KVC_GLOBAL T* gptr(T* p) {
  return (KVC_GLOBAL T*)p;
}
template <typename T>
__device__ __forceinline__ KVC_GLOBAL T* gptr_from_int(uint64_t addr) {
  return (KVC_GLOBAL T*)addr;
}

// 16-bit float words packed two per dword, low half first in memory.
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float fp16_lo(uint32_t w) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w & 0xffffu)));
}
__device__ __forceinline__ float fp16_hi(uint32_t w) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w >> 16)));
}

template <typename T>
struct Unpack;

struct Bf16Tag {};
struct Fp16Tag {};

template <>
struct Unpack<Bf16Tag> {
  __device__ __forceinline__ static float lo(uint32_t w) { return bf16_lo(w); }
  __device__ __forceinline__ static float hi(uint32_t w) { return bf16_hi(w); }
};
template <>
struct Unpack<Fp16Tag> {
  __device__ __forceinline__ static float lo(uint32_t w) { return fp16_lo(w); }
  __device__ __forceinline__ static float hi(uint32_t w) { return fp16_hi(w); }
};

// NaN-propagating maximum (torch.amax / torch.maximum semantics).
__device__ __forceinline__ float max_nan(float a, float b) {
  if (a != a) return a;
  if (b != b) return b;
  return a > b ? a : b;
}

// Cross-lane sum inside groups of `width` lanes (width a power of two <= 64).
// Widths up to 16 use DPP row permutations; wider ones fall back to shuffles.
__device__ __forceinline__ float dpp_quad_xor1(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));
}
__device__ __forceinline__ float dpp_quad_xor2(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));
}
__device__ __forceinline__ float dpp_row_half_mirror(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false));
}
__device__ __forceinline__ float dpp_row_mirror(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false));
}

// After step k every lane of an aligned group of 2^k lanes holds the group sum:
// xor1/xor2 sum quads; half-mirror (lane i <-> 7-i) adds the other quad of an
// 8-lane half-row; mirror (i <-> 15-i) adds the other half of a 16-lane row.
__device__ __forceinline__ float group_sum(float v, int width) {
  if (width >= 2) v += dpp_quad_xor1(v);
  if (width >= 4) v += dpp_quad_xor2(v);
  if (width >= 8) v += dpp_row_half_mirror(v);
  if (width >= 16) v += dpp_row_mirror(v);
  if (width >= 32) v += __shfl_xor(v, 16);
  if (width >= 64) v += __shfl_xor(v, 32);
  return v;
}

// Order-preserving map from float bits to unsigned keys (larger float ->
// larger key; NaN with clear sign sorts above +inf as torch.topk ranks it).
__device__ __forceinline__ uint32_t float_key(float f) {
  uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

}  // namespace kvc
