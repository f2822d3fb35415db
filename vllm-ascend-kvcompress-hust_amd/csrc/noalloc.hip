// kvc_score_paged_noalloc: kvc_score_paged followed by kvc_head_stats with the
// scorer's scratch (folded weights and per-tile float64 partial sums) in a
// file-scope device array instead of a caller workspace, for callers that
// cannot allocate device memory (HIP graph capture, serving loops that forbid
// allocation).  The kernels are the ones kvc_score_paged and kvc_head_stats
// launch; only where the scratch lives differs.
//
// The array is a device symbol: its name in host code is a host-side stand-in,
// not a device address.  The device address is taken once per device with
// hipGetSymbolAddress, with that device current, on the first call on it, and
// kept; every launch receives that address.

#include <mutex>

#include "score_internal.h"

namespace kvc {
namespace {

constexpr size_t kNoallocScratchBytes = size_t{64} << 20;  // 64 MiB per device
constexpr int kNoallocMaxDevices = 64;

__device__ __align__(256) unsigned char scratch[kNoallocScratchBytes];

std::mutex g_scratch_mutex;
void* g_scratch_ptr[kNoallocMaxDevices] = {};

// Device address of `scratch` on the device `stream` runs on, which must be the
// current device.
int scratch_address(hipStream_t stream, void** out) {
  int current = -1;
  hipError_t e = hipGetDevice(&current);
  if (e != hipSuccess) return fail(static_cast<int>(e), "kvc_score_paged_noalloc: hipGetDevice: %s", hipGetErrorString(e));
  int stream_device = current;
  if (stream != nullptr) {
    e = hipStreamGetDevice(stream, &stream_device);
    if (e != hipSuccess)
      return fail(static_cast<int>(e), "kvc_score_paged_noalloc: hipStreamGetDevice: %s", hipGetErrorString(e));
  }
  if (stream_device != current)
    return fail(KVC_EINVAL, "kvc_score_paged_noalloc: the stream belongs to device %d, the current device is %d",
                stream_device, current);
  if (current < 0 || current >= kNoallocMaxDevices)
    return fail(KVC_EINVAL, "kvc_score_paged_noalloc: device %d beyond the %d this library tracks", current,
                kNoallocMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[current] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return fail(e != hipSuccess ? static_cast<int>(e) : KVC_EINVAL,
                  "kvc_score_paged_noalloc: hipGetSymbolAddress of the scratch array: %s", hipGetErrorString(e));
    g_scratch_ptr[current] = p;
  }
  *out = g_scratch_ptr[current];
  return 0;
}

}  // namespace
}  // namespace kvc

using namespace kvc;

extern "C" int kvc_score_paged_noalloc(kvc_stream_t stream, int dtype, int n_layers, const uint64_t* k_layer_ptrs,
                                       int64_t num_pages, int64_t page_stride, int kv_heads, int head_dim,
                                       int rotary_dim, int qpk, int rope_style, int n_seq, int max_seq_len,
                                       const int32_t* seq_lens, const int64_t* token_offsets,
                                       const int64_t* block_offsets, const int64_t* block_ids, const float* q_real,
                                       const float* q_imag, const float* freq_scale, const float* extra_coef,
                                       const float* q_pass, const float* phase_cos, const float* phase_sin,
                                       int64_t phase_seq_stride, float* raw, int64_t raw_layer_stride,
                                       int64_t raw_token_stride, int64_t raw_head_stride, float* mean, float* var) {
  // Size and output checks come first: nothing is launched for a call that is
  // going to be rejected.
  const size_t need = kvc_score_workspace_bytes(n_layers, kv_heads, head_dim, rotary_dim, qpk, n_seq, max_seq_len);
  if (need == 0) return fail(KVC_EINVAL, "kvc_score_paged_noalloc: unsupported shape");
  if (need > kNoallocScratchBytes)
    return fail(KVC_EINVAL,
                "kvc_score_paged_noalloc: this batch needs %zu bytes of scratch, more than the %zu bytes (64 MiB) "
                "of the static scratch; use kvc_score_paged with a workspace",
                need, kNoallocScratchBytes);
  if (!mean || !var) return fail(KVC_EINVAL, "kvc_score_paged_noalloc: null pointer");
  hipStream_t st = as_stream(stream);
  void* ws = nullptr;
  if (int rc = scratch_address(st, &ws)) return rc;
  // Nothing in the scratch has to start at zero: the fold writes every weight
  // the scorer reads, the scorer writes the partial sums of every tile that
  // holds tokens, and kvc_head_stats reads only those tiles.
  if (int rc = kvc_score_paged(stream, dtype, n_layers, k_layer_ptrs, num_pages, page_stride, kv_heads, head_dim,
                               rotary_dim, qpk, rope_style, n_seq, max_seq_len, seq_lens, token_offsets, block_offsets,
                               block_ids, q_real, q_imag, freq_scale, extra_coef, q_pass, phase_cos, phase_sin,
                               phase_seq_stride, raw, raw_layer_stride, raw_token_stride, raw_head_stride, ws,
                               kNoallocScratchBytes))
    return rc;
  return kvc_head_stats(stream, n_layers, kv_heads, head_dim, rotary_dim, qpk, n_seq, max_seq_len, seq_lens, ws,
                        kNoallocScratchBytes, mean, var);
}
