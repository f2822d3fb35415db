// HBM bandwidth probes used to state the achievable ceilings next to the
// roofline figures: streaming read, write and copy of 16-byte words with a
// grid-stride loop, optionally with non-temporal hints (kinds 0-2), and a
// block-contiguous, software-pipelined copy (kind 3).

#include "kvc_common.h"

namespace kvc {
namespace {

typedef uint32_t w128 __attribute__((ext_vector_type(4)));

template <int NT>
__global__ __launch_bounds__(256) void probe_read(const w128* __restrict__ src, int64_t n, uint32_t* sink) {
  uint32_t acc = 0;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += stride * 4) {
    w128 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t j = i + u * stride;
      v[u] = j < n ? (NT ? __builtin_nontemporal_load(src + j) : src[j]) : w128{0, 0, 0, 0};
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  if (acc == 0x9E3779B9u) sink[0] = acc;  // data-dependent store keeps the loads
}

template <int NT>
__global__ __launch_bounds__(256) void probe_write(w128* __restrict__ dst, int64_t n) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += stride) {
    const w128 v = {static_cast<uint32_t>(i), 1u, 2u, 3u};
    if (NT)
      __builtin_nontemporal_store(v, dst + i);
    else
      dst[i] = v;
  }
}

template <int NT>
__global__ __launch_bounds__(256) void probe_copy(const w128* __restrict__ src, w128* __restrict__ dst, int64_t n) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += stride * 4) {
    w128 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t j = i + u * stride;
      if (j < n) v[u] = NT ? __builtin_nontemporal_load(src + j) : src[j];
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t j = i + u * stride;
      if (j < n) {
        if (NT)
          __builtin_nontemporal_store(v[u], dst + j);
        else
          dst[j] = v[u];
      }
    }
  }
}

// Block-contiguous copy: workgroup g copies words [g*per_wg, (g+1)*per_wg) in
// steps of 8 words per thread, loading the next step before storing the
// current one (512-thread workgroups).
constexpr int kChunkThreads = 512;
constexpr int kChunkUnroll = 8;

__global__ __launch_bounds__(kChunkThreads) void probe_copy_chunked(const w128* __restrict__ src,
                                                                    w128* __restrict__ dst, int64_t n,
                                                                    int64_t per_wg) {
  const int64_t begin = static_cast<int64_t>(blockIdx.x) * per_wg;
  const int64_t end = begin + per_wg < n ? begin + per_wg : n;
  const int64_t step = static_cast<int64_t>(kChunkUnroll) * kChunkThreads;
  w128 a[kChunkUnroll], b[kChunkUnroll];
  auto load = [&](int64_t base, w128 (&v)[kChunkUnroll]) {
#pragma unroll
    for (int u = 0; u < kChunkUnroll; ++u) {
      const int64_t j = base + u * kChunkThreads + threadIdx.x;
      if (j < end) v[u] = __builtin_nontemporal_load(src + j);
    }
  };
  auto store = [&](int64_t base, const w128 (&v)[kChunkUnroll]) {
#pragma unroll
    for (int u = 0; u < kChunkUnroll; ++u) {
      const int64_t j = base + u * kChunkThreads + threadIdx.x;
      if (j < end) __builtin_nontemporal_store(v[u], dst + j);
    }
  };
  int64_t base = begin;
  load(base, a);
  for (; base < end; base += 2 * step) {
    load(base + step, b);
    store(base, a);
    if (base + step >= end) break;
    load(base + 2 * step, a);
    store(base + step, b);
  }
}

}  // namespace
}  // namespace kvc

using namespace kvc;

extern "C" int kvc_bandwidth_probe(kvc_stream_t stream, int kind, int nontemporal, const void* src, void* dst,
                                   int64_t bytes, int blocks) {
  if (bytes <= 0 || bytes % 16 != 0 || blocks <= 0 || kind < 0 || kind > 3)
    return fail(KVC_EINVAL, "kvc_bandwidth_probe: bad arguments");
  if ((kind != 1 && !src) || !dst) return fail(KVC_EINVAL, "kvc_bandwidth_probe: null pointer");
  const int64_t n = bytes / 16;
  hipStream_t st = as_stream(stream);
  const w128* s = static_cast<const w128*>(src);
  w128* d = static_cast<w128*>(dst);
  if (kind == 0) {
    if (nontemporal) probe_read<1><<<blocks, 256, 0, st>>>(s, n, static_cast<uint32_t*>(dst));
    else probe_read<0><<<blocks, 256, 0, st>>>(s, n, static_cast<uint32_t*>(dst));
  } else if (kind == 1) {
    if (nontemporal) probe_write<1><<<blocks, 256, 0, st>>>(d, n);
    else probe_write<0><<<blocks, 256, 0, st>>>(d, n);
  } else if (kind == 2) {
    if (nontemporal) probe_copy<1><<<blocks, 256, 0, st>>>(s, d, n);
    else probe_copy<0><<<blocks, 256, 0, st>>>(s, d, n);
  } else {
    probe_copy_chunked<<<blocks, kChunkThreads, 0, st>>>(s, d, n, ceil_div(n, blocks));
  }
  return launch_status("kvc_bandwidth_probe");
}
