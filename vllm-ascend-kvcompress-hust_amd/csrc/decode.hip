// Decode-side consumers of a compacted cache: physical positions, slot
// mapping and attention lengths.
//
// Compaction keeps semantic RoPE positions monotonic; only where a token's K/V
// row lives moves.  A request compacted from semantic length S to physical
// length P carries offset S - P (pkg/provider.py:52-54), and every later token
// of that request is written at physical position semantic - offset
// (shift_positions, tri/kernels.py:35-47, used by the slot-mapping hook
// pkg/provider.py:687-705 ahead of the host's compute_slot_mapping).  The
// attention lengths shrink by the same offset (pkg/provider.py:707-728).
//
// All three are integer gathers over a few thousand entries per step: one
// thread per entry, no LDS.

#include "kvc_common.h"

namespace kvc {
namespace {

constexpr int kDecodeThreads = 256;

__device__ __forceinline__ int64_t load_index(const void* p, int bytes, int64_t i) {
  return bytes == 4 ? static_cast<int64_t>(static_cast<const int32_t*>(p)[i]) : static_cast<const int64_t*>(p)[i];
}

__global__ __launch_bounds__(kDecodeThreads) void shift_positions_kernel(const int64_t* __restrict__ positions,
                                                                         const void* __restrict__ request_indices,
                                                                         int index_bytes,
                                                                         const int64_t* __restrict__ offsets, int64_t n,
                                                                         int64_t* __restrict__ out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kDecodeThreads + threadIdx.x;
  if (i >= n) return;
  out[i] = positions[i] - offsets[load_index(request_indices, index_bytes, i)];
}

// One workgroup per request (grid-stride over requests); the request's tokens
// are [query_start_loc[r], query_start_loc[r+1]).  Tokens past the last
// request (graph padding) get -1, as do positions outside the block table.
__global__ __launch_bounds__(kDecodeThreads) void slot_mapping_kernel(
    int num_reqs, const int32_t* __restrict__ query_start_loc, const int64_t* __restrict__ positions,
    const int64_t* __restrict__ offsets, const int32_t* __restrict__ block_table, int64_t table_stride,
    int max_blocks, int block_size, int64_t num_tokens, int64_t* __restrict__ slot_mapping,
    int64_t* __restrict__ physical_out) {
  for (int r = blockIdx.x; r <= num_reqs; r += gridDim.x) {
    if (r == num_reqs) {
      // Padding tokens after the last request.
      for (int64_t i = query_start_loc[num_reqs] + threadIdx.x; i < num_tokens; i += kDecodeThreads) {
        slot_mapping[i] = -1;
        if (physical_out) physical_out[i] = positions[i];
      }
      continue;
    }
    const int64_t begin = query_start_loc[r];
    const int64_t end = query_start_loc[r + 1];
    const int64_t off = offsets ? offsets[r] : 0;
    const int32_t* row = block_table + static_cast<int64_t>(r) * table_stride;
    for (int64_t i = begin + threadIdx.x; i < end && i < num_tokens; i += kDecodeThreads) {
      const int64_t p = positions[i] - off;
      const int64_t blk = p >= 0 ? p / block_size : -1;
      int64_t slot = -1;
      if (blk >= 0 && blk < max_blocks) {
        const int64_t page = row[blk];
        if (page >= 0) slot = page * block_size + (p - blk * block_size);
      }
      slot_mapping[i] = slot;
      if (physical_out) physical_out[i] = p;
    }
  }
}

template <typename T>
__global__ __launch_bounds__(kDecodeThreads) void shift_lengths_kernel(T* __restrict__ seq_lens,
                                                                       const int64_t* __restrict__ offsets,
                                                                       int num_reqs) {
  const int r = blockIdx.x * kDecodeThreads + threadIdx.x;
  if (r >= num_reqs) return;
  seq_lens[r] = static_cast<T>(static_cast<int64_t>(seq_lens[r]) - offsets[r]);
}

}  // namespace
}  // namespace kvc

using namespace kvc;

extern "C" int kvc_shift_positions(kvc_stream_t stream, const int64_t* positions, const void* request_indices,
                                   int index_bytes, const int64_t* request_offsets, int64_t n,
                                   int64_t* output) {
  if (n < 0) return fail(KVC_EINVAL, "kvc_shift_positions: n must be non-negative");
  if (index_bytes != 4 && index_bytes != 8)
    return fail(KVC_EINVAL, "kvc_shift_positions: index_bytes must be 4 or 8");
  if (n == 0) return 0;
  if (!positions || !request_indices || !request_offsets || !output)
    return fail(KVC_EINVAL, "kvc_shift_positions: null pointer");
  shift_positions_kernel<<<static_cast<unsigned>(ceil_div(n, kDecodeThreads)), kDecodeThreads, 0,
                           as_stream(stream)>>>(positions, request_indices, index_bytes, request_offsets, n,
                                                output);
  return launch_status("kvc_shift_positions");
}

extern "C" int kvc_physical_slot_mapping(kvc_stream_t stream, int num_reqs, const int32_t* query_start_loc,
                                         const int64_t* positions, const int64_t* request_offsets,
                                         const int32_t* block_table, int64_t block_table_stride, int max_blocks,
                                         int block_size, int64_t num_tokens, int64_t* slot_mapping,
                                         int64_t* physical_positions) {
  if (num_reqs < 0 || num_tokens < 0 || max_blocks < 0 || block_size <= 0)
    return fail(KVC_EINVAL, "kvc_physical_slot_mapping: bad sizes");
  if (block_table_stride < max_blocks)
    return fail(KVC_EINVAL, "kvc_physical_slot_mapping: block_table_stride < max_blocks");
  if (num_tokens == 0) return 0;
  if (!query_start_loc || !positions || !slot_mapping || (num_reqs > 0 && !block_table))
    return fail(KVC_EINVAL, "kvc_physical_slot_mapping: null pointer");
  const unsigned blocks = static_cast<unsigned>(num_reqs + 1 < 4096 ? num_reqs + 1 : 4096);
  slot_mapping_kernel<<<blocks, kDecodeThreads, 0, as_stream(stream)>>>(
      num_reqs, query_start_loc, positions, request_offsets, block_table, block_table_stride, max_blocks,
      block_size, num_tokens, slot_mapping, physical_positions);
  return launch_status("kvc_physical_slot_mapping");
}

extern "C" int kvc_shift_lengths(kvc_stream_t stream, void* seq_lens, int elem_bytes, const int64_t* request_offsets,
                                 int num_reqs) {
  if (num_reqs < 0) return fail(KVC_EINVAL, "kvc_shift_lengths: num_reqs must be non-negative");
  if (elem_bytes != 4 && elem_bytes != 8) return fail(KVC_EINVAL, "kvc_shift_lengths: elem_bytes must be 4 or 8");
  if (num_reqs == 0) return 0;
  if (!seq_lens || !request_offsets) return fail(KVC_EINVAL, "kvc_shift_lengths: null pointer");
  const unsigned blocks = static_cast<unsigned>(ceil_div(num_reqs, kDecodeThreads));
  if (elem_bytes == 4)
    shift_lengths_kernel<int32_t><<<blocks, kDecodeThreads, 0, as_stream(stream)>>>(static_cast<int32_t*>(seq_lens),
                                                                                     request_offsets, num_reqs);
  else
    shift_lengths_kernel<int64_t><<<blocks, kDecodeThreads, 0, as_stream(stream)>>>(static_cast<int64_t*>(seq_lens),
                                                                                     request_offsets, num_reqs);
  return launch_status("kvc_shift_lengths");
}
