// KV compaction on CDNA4: kept K/V rows -> destination rows, all layers in one launch.
//
// Row i (< budget) of sequence b's destination receives source row keep[b][i].
// A row is the kv_heads*head_dim elements of one token, contiguous inside its
// page (reference cache layout [pages][128][kv_heads][head_dim]).  Rows are
// moved in `Chunk`-sized words by a thread layout of (row lane, column):
// `slice_w` consecutive threads cover a slice of one row, so every wave
// instruction reads and writes whole 128-byte lines.
//
// Private mode (destination pages disjoint from the source pages), two forms:
//  * planned (a workspace is given and the batch has at most kPlanMaxSeqs
//    sequences): one launch resolves every kept row once (keep index -> source
//    page -> byte offset, and the destination offset) into the workspace, then
//    a second launch moves one layer's rows per workgroup, reading the
//    offsets instead of chasing the indices, in the caller's order: layer
//    after layer (the workgroups in flight at any time touch one or two
//    layers' pages, so the translation working set stays small whatever the
//    physical placement of the pool: moving all layers per workgroup touches
//    every layer's buffers at once and ran 4.2-5.3 ms on the Qwen2.5-14B
//    16 x 16384 shape depending on the placement, the layer-major form
//    4.15-4.47 ms on the same buffers) or every layer's workgroups
//    interleaved (faster in some placements, slower in others; see
//    compact_layer_kernel);
//  * walked: a workgroup owns a tile of rows x one column slice of one
//    sequence, resolves the rows' offsets once and walks every layer, loading
//    the K and V words of the tile together before storing them.  Used
//    without a workspace and for large batches (201 sequences: 26.6 ms against
//    27.9 ms for the layer-major form).
//
// In-place mode (destinations are the sequence's own front pages, rows
// [0, budget)): keep is strictly increasing, so keep[j] >= j, and the rows
// split at J0, the first j with keep[j] >= budget:
//  * hazard rows j < J0 read a row below the budget, which another
//    destination may overwrite (row r is written by destination r >= j).  A
//    workgroup owns one column slice of one (layer, sequence) and walks these
//    rows in ascending tiles: every load of a tile (K and V) completes before
//    a workgroup barrier, then the tile's stores go out.  A row read by tile T
//    lies at index >= the first row of tile T, so it is overwritten, if at
//    all, by tile T itself (after the barrier) or by a later tile.  The walk
//    stops at the first tile that starts at or after J0.
//  * safe rows j >= J0 read rows >= budget, which no destination writes, and
//    write rows in [J0, budget), which only hazard rows read.  Once the walk
//    has finished they move with no ordering at all: through the planned
//    layer-major copy when a workspace is given (at most kPlanMaxSeqs
//    sequences; the plan marks hazard rows as moving nothing), otherwise
//    through the private-mode kernel over the same table.  The planned form
//    moved the safe rows of the Qwen2.5-14B 4 x 131072 shape (48 layers,
//    4608 kept rows each) in 1.34 ms against 1.44 ms for the walked one.
// Column slices are disjoint bytes, so slices run in parallel.  Rows whose
// source and destination coincide are skipped.

#include "kvc_common.h"

namespace kvc {
namespace {

// Row-parallel kernel: one row per thread, 256-thread workgroups.  Timed on
// fresh data in one allocation, against 512 threads: 4.27 vs 4.29 ms
// (Qwen2.5-14B shape, 16 x 4096 kept rows of 2 KB, 48 layers), 1.43 vs
// 1.50 ms (4 x 4608 rows kept of 131072, in place), 0.286 vs 0.296 ms
// (Qwen3.5 shape, 1 KB rows); 2 or 4 rows per thread and 1024 threads were
// slower on all three, 128 threads level with 256.
// In-place mode walks its tiles in order behind a barrier; 2 rows per thread
// at 512 threads measured 0.85 ms on the 4 x 131072-token shape (48 layers,
// 4608 kept rows) against 1.32 ms for 8 rows at 256 threads.

constexpr int kCopyThreads = 256;
// Planned private mode: 128-thread workgroups (one 2 KB row per workgroup; 128
// and 256 threads measured level, 512 and 1024 slower) for batches of at most
// kPlanMaxSeqs sequences.
constexpr int kPlanThreads = 128;
constexpr int kPlanMaxSeqs = 32;
constexpr int kCopyUnroll = 1;  // rows per thread per tile (private mode)
constexpr int kInplaceThreads = 512;
constexpr int kInplaceUnroll = 2;  // rows per thread per tile (in place)

// Native vector words (the HIP_vector_type structs would be kept in scratch).
typedef uint32_t w128 __attribute__((ext_vector_type(4)));
typedef uint32_t w64 __attribute__((ext_vector_type(2)));

struct CompactArgs {
  const uint64_t* k_ptrs;
  const uint64_t* v_ptrs;
  int n_layers;
  int n_seq;
  int64_t num_pages;
  int64_t page_stride_bytes;
  int64_t row_bytes;
  int64_t row_chunks;    // row_bytes / sizeof(Chunk)
  int slice_shift;       // log2(chunks per column slice)
  int n_slices;
  int budget;
  const int32_t* seq_lens;
  const int64_t* src_off;
  const int64_t* src_ids;
  const int64_t* dst_off;
  const int64_t* dst_ids;
  const int64_t* keep;
  int64_t keep_stride;
  int rows;              // kRowsAll, or the in-place halves kRowsHazard / kRowsSafe
};

constexpr int kRowsAll = 0;
constexpr int kRowsHazard = 1;  // keep[i] < budget (in place, ordered walk)
constexpr int kRowsSafe = 2;    // keep[i] >= budget (in place, any order)

// Streaming word access; the non-temporal forms mark lines for early eviction.
template <typename Chunk>
__device__ __forceinline__ Chunk load_word(KVC_GLOBAL const char* p) {
  return __builtin_nontemporal_load(reinterpret_cast<KVC_GLOBAL const Chunk*>(p));
}
template <typename Chunk>
__device__ __forceinline__ void store_word(KVC_GLOBAL char* p, Chunk v) {
  __builtin_nontemporal_store(v, reinterpret_cast<KVC_GLOBAL Chunk*>(p));
}

__device__ __forceinline__ int64_t page_of(const int64_t* table, int64_t n_entries, int64_t row,
                                           int64_t num_pages) {
  const int64_t blk = row >> kBlockShift;
  if (row < 0 || blk >= n_entries) return -1;
  const int64_t p = table[blk];
  return (p >= 0 && p < num_pages) ? p : -1;
}

// Byte offsets (inside one layer's buffer) of the source and destination word
// of row `i`, or -1 when the row is out of range, unmapped or already in place.
struct RowMove {
  int64_t src, dst;
};

__device__ __forceinline__ RowMove resolve_row(const CompactArgs& a, const int64_t* sbt, int64_t n_src,
                                               const int64_t* dbt, int64_t n_dst, const int64_t* kp,
                                               int64_t n_tokens, int64_t i, int64_t word_off,
                                               bool col_ok) {
  RowMove m{-1, -1};
  if (!col_ok || i >= a.budget) return m;
  const int64_t src_row = kp[i];
  if (src_row < 0 || src_row >= n_tokens) return m;
  if (a.rows != kRowsAll && (src_row < a.budget) != (a.rows == kRowsHazard)) return m;
  const int64_t sp = page_of(sbt, n_src, src_row, a.num_pages);
  const int64_t dp = page_of(dbt, n_dst, i, a.num_pages);
  if (sp < 0 || dp < 0) return m;
  const int64_t so = sp * a.page_stride_bytes + (src_row & (kBlockSize - 1)) * a.row_bytes + word_off;
  const int64_t dof = dp * a.page_stride_bytes + (i & (kBlockSize - 1)) * a.row_bytes + word_off;
  if (so == dof) return m;
  m.src = so;
  m.dst = dof;
  return m;
}

// Rows `tile` of sequence `b` as (source, destination) byte offsets of the
// thread's word, resolved once for every layer.
template <int U>
__device__ __forceinline__ void resolve_tile(const CompactArgs& a, int b, int64_t tile, int tile_rows,
                                             int rows_per_step, int row_lane, int64_t word_off, bool col_ok,
                                             RowMove (&mv)[U]) {
  const int64_t* sbt = a.src_ids + a.src_off[b];
  const int64_t n_src = a.src_off[b + 1] - a.src_off[b];
  const int64_t* dbt = a.dst_ids + a.dst_off[b];
  const int64_t n_dst = a.dst_off[b + 1] - a.dst_off[b];
  const int64_t* kp = a.keep + static_cast<int64_t>(b) * a.keep_stride;
  const int64_t n_tokens = a.seq_lens[b];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t i = tile * tile_rows + u * rows_per_step + row_lane;
    mv[u] = resolve_row(a, sbt, n_src, dbt, n_dst, kp, n_tokens, i, word_off, col_ok);
  }
}

// Row-parallel kernel (private mode, and the safe rows of in-place mode): a
// workgroup moves the K and V words of one row tile x one column slice of one
// sequence through every layer.
template <typename Chunk>
__global__ __launch_bounds__(kCopyThreads) void compact_private_kernel(CompactArgs a) {
  // One-dimensional grid, sequence fastest: the workgroups resident at a time
  // spread over every sequence's pages (3% faster on the Qwen2.5-14B shape
  // than tile-major order, which keeps them inside one or two sequences).
  const int b = static_cast<int>(blockIdx.x % a.n_seq);
  const int64_t rest = blockIdx.x / a.n_seq;
  const int slice = static_cast<int>(rest % a.n_slices);
  const int tile = static_cast<int>(rest / a.n_slices);
  const int slice_w = 1 << a.slice_shift;
  const int rows_per_step = kCopyThreads >> a.slice_shift;
  const int tile_rows = rows_per_step * kCopyUnroll;
  const int col = threadIdx.x & (slice_w - 1);
  const int row_lane = threadIdx.x >> a.slice_shift;
  const int64_t chunk = static_cast<int64_t>(slice) * slice_w + col;
  const bool col_ok = chunk < a.row_chunks;
  const int64_t word_off = chunk * static_cast<int64_t>(sizeof(Chunk));

  RowMove mv[kCopyUnroll];
  resolve_tile(a, b, tile, tile_rows, rows_per_step, row_lane, word_off, col_ok, mv);

  for (int layer = 0; layer < a.n_layers; ++layer) {
    KVC_GLOBAL char* kb = gptr_from_int<char>(a.k_ptrs[layer]);
    KVC_GLOBAL char* vb = gptr_from_int<char>(a.v_ptrs[layer]);
    Chunk kv[kCopyUnroll], vv[kCopyUnroll];
#pragma unroll
    for (int u = 0; u < kCopyUnroll; ++u) {
      if (mv[u].src >= 0) {
        kv[u] = load_word<Chunk>(kb + mv[u].src);
        vv[u] = load_word<Chunk>(vb + mv[u].src);
      }
    }
#pragma unroll
    for (int u = 0; u < kCopyUnroll; ++u) {
      if (mv[u].src >= 0) {
        store_word<Chunk>(kb + mv[u].dst, kv[u]);
        store_word<Chunk>(vb + mv[u].dst, vv[u]);
      }
    }
  }
}


// Planned private mode, first launch: the byte offsets (inside one layer's
// buffer) of every kept row's source and destination, -1 for rows that move
// nothing, as plan[2*(b*budget + i)] and plan[2*(b*budget + i) + 1].
__global__ void compact_plan_kernel(CompactArgs a, int64_t* __restrict__ plan) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= static_cast<int64_t>(a.n_seq) * a.budget) return;
  const int b = static_cast<int>(idx / a.budget);
  const int64_t i = idx - static_cast<int64_t>(b) * a.budget;
  const int64_t* sbt = a.src_ids + a.src_off[b];
  const int64_t n_src = a.src_off[b + 1] - a.src_off[b];
  const int64_t* dbt = a.dst_ids + a.dst_off[b];
  const int64_t n_dst = a.dst_off[b + 1] - a.dst_off[b];
  const int64_t* kp = a.keep + static_cast<int64_t>(b) * a.keep_stride;
  const RowMove m = resolve_row(a, sbt, n_src, dbt, n_dst, kp, a.seq_lens[b], i, 0, true);
  plan[2 * idx] = m.src;
  plan[2 * idx + 1] = m.dst;
}

// Store policy of the layer-major copy: device-scope non-temporal (sc1 nt)
// 16-byte buffer stores.  On the Qwen2.5-14B 16 x 16384 pool the copy ran
// 4.385 - 4.397 ms with them against 4.467 - 4.480 ms with the plain
// non-temporal global store, in three placements; the interleaved order ran
// 0.8 - 1.2% slower with them and keeps the global form, as do buffers whose
// extent needs offsets past 32 bits.  The load policy made no difference.
constexpr int kBufferSc1Nt = 16 | 2;  // cache-policy bits: sc1 = 16, nt = 2

__device__ __forceinline__ __amdgpu_buffer_rsrc_t layer_rsrc(KVC_GLOBAL char* base) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)(uintptr_t)base, 0, 0xFFFFFFFFu, 0x00020000);
}

// Planned mode, second launch: a workgroup moves the K and V words of one row
// tile x one column slice of one sequence in one layer.  Grid order, fastest
// first: layer-major = (sequence, slice, tile, layer): the layers one after
// the other; interleaved = (layer, slice, tile, sequence): every layer's
// buffers in flight at once, a sequence at a time.  Of the six nestings of
// (sequence, row tile, layer) timed over five placements of the Qwen2.5-14B
// pool, these were the best two: layer-major 4.37 - 4.49 ms in every one,
// interleaved 4.12 - 4.24 ms in three and 4.59 - 4.77 ms in two; (layer,
// sequence, tile) followed the interleaved order 0.05 - 0.26 ms behind it.
template <typename Chunk, bool SC1_STORES = false>
__global__ __launch_bounds__(kPlanThreads) void compact_layer_kernel(CompactArgs a, const int64_t* __restrict__ plan,
                                                                     int64_t per_layer, bool interleaved) {
  int layer, b;
  int64_t rest;  // slice + n_slices * tile
  if (interleaved) {
    const int64_t per_seq = per_layer / a.n_seq;
    layer = static_cast<int>(blockIdx.x % a.n_layers);
    const int64_t x = blockIdx.x / a.n_layers;
    rest = x % per_seq;
    b = static_cast<int>(x / per_seq);
  } else {
    layer = static_cast<int>(blockIdx.x / per_layer);
    const int64_t bx = blockIdx.x - static_cast<int64_t>(layer) * per_layer;
    b = static_cast<int>(bx % a.n_seq);
    rest = bx / a.n_seq;
  }
  const int slice = static_cast<int>(rest % a.n_slices);
  const int64_t tile = rest / a.n_slices;
  const int slice_w = 1 << a.slice_shift;
  const int col = threadIdx.x & (slice_w - 1);
  const int64_t chunk = static_cast<int64_t>(slice) * slice_w + col;
  const int64_t i = tile * (kPlanThreads >> a.slice_shift) + (threadIdx.x >> a.slice_shift);
  if (chunk >= a.row_chunks || i >= a.budget) return;
  const int64_t* pp = plan + 2 * (static_cast<int64_t>(b) * a.budget + i);
  const int64_t src = pp[0];
  if (src < 0) return;
  const int64_t dst = pp[1];
  const int64_t word_off = chunk * static_cast<int64_t>(sizeof(Chunk));
  KVC_GLOBAL char* kb = gptr_from_int<char>(a.k_ptrs[layer]);
  KVC_GLOBAL char* vb = gptr_from_int<char>(a.v_ptrs[layer]);
  const Chunk kv = load_word<Chunk>(kb + src + word_off);
  const Chunk vv = load_word<Chunk>(vb + src + word_off);
  if constexpr (SC1_STORES) {
    static_assert(sizeof(Chunk) == 16, "16-byte words only");
    const unsigned off = static_cast<unsigned>(dst + word_off);  // the launcher checked the extent
    __builtin_amdgcn_raw_buffer_store_b128(kv, layer_rsrc(kb), off, 0, kBufferSc1Nt);
    __builtin_amdgcn_raw_buffer_store_b128(vv, layer_rsrc(vb), off, 0, kBufferSc1Nt);
  } else {
    store_word<Chunk>(kb + dst + word_off, kv);
    store_word<Chunk>(vb + dst + word_off, vv);
  }
}

// Whether the walk reaches tile `tile`: the tile starts inside the budget at
// a hazard row (keep is increasing, so no hazard row follows a safe one).
// The same value in every thread of the workgroup.
__device__ __forceinline__ bool hazard_tile(const CompactArgs& a, const int64_t* kp, int tile, int tile_rows) {
  const int64_t first = static_cast<int64_t>(tile) * tile_rows;
  return first < a.budget && kp[first] < a.budget;
}

// Hazard rows of tile `tile`, moved in place inside one sequence's own pages.
template <int U>
__device__ __forceinline__ void resolve_inplace(const CompactArgs& a, int b, int tile, bool live, int tile_rows,
                                                int rows_per_step, int row_lane, int64_t word_off, bool col_ok,
                                                RowMove (&mv)[U]) {
  const int64_t* sbt = a.src_ids + a.src_off[b];
  const int64_t n_src = a.src_off[b + 1] - a.src_off[b];
  const int64_t* kp = a.keep + static_cast<int64_t>(b) * a.keep_stride;
  const int64_t n_tokens = a.seq_lens[b];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t i = static_cast<int64_t>(tile) * tile_rows + u * rows_per_step + row_lane;
    mv[u] = live ? resolve_row(a, sbt, n_src, sbt, n_src, kp, n_tokens, i, word_off, col_ok) : RowMove{-1, -1};
  }
}

// In-place mode, hazard rows: a workgroup owns one column slice of one
// (layer, sequence) and walks the hazard rows in ascending tiles.  All loads
// of a tile complete before the workgroup barrier, then its stores go out.
// The rows of the next tile are resolved (keep index -> page -> offset) while
// the current tile's words are in flight; keep and the block tables are never
// written here.
template <typename Chunk>
__global__ __launch_bounds__(kInplaceThreads) void compact_inplace_kernel(CompactArgs a) {
  const int b = blockIdx.y;
  const int layer = blockIdx.z;
  const int slice = blockIdx.x;
  KVC_GLOBAL char* kb = gptr_from_int<char>(a.k_ptrs[layer]);
  KVC_GLOBAL char* vb = gptr_from_int<char>(a.v_ptrs[layer]);
  const int slice_w = 1 << a.slice_shift;
  const int rows_per_step = kInplaceThreads >> a.slice_shift;
  const int tile_rows = rows_per_step * kInplaceUnroll;
  const int col = threadIdx.x & (slice_w - 1);
  const int row_lane = threadIdx.x >> a.slice_shift;
  const int64_t chunk = static_cast<int64_t>(slice) * slice_w + col;
  const bool col_ok = chunk < a.row_chunks;
  const int64_t word_off = chunk * static_cast<int64_t>(sizeof(Chunk));
  const int64_t* kp = a.keep + static_cast<int64_t>(b) * a.keep_stride;

  bool live = hazard_tile(a, kp, 0, tile_rows);
  RowMove mv[kInplaceUnroll];
  resolve_inplace(a, b, 0, live, tile_rows, rows_per_step, row_lane, word_off, col_ok, mv);
  for (int tile = 0; live; ++tile) {
    Chunk kv[kInplaceUnroll], vv[kInplaceUnroll];
#pragma unroll
    for (int u = 0; u < kInplaceUnroll; ++u) {
      if (mv[u].src >= 0) {
        kv[u] = *reinterpret_cast<KVC_GLOBAL const Chunk*>(kb + mv[u].src);
        vv[u] = *reinterpret_cast<KVC_GLOBAL const Chunk*>(vb + mv[u].src);
      }
    }
    const bool live_next = hazard_tile(a, kp, tile + 1, tile_rows);
    RowMove next[kInplaceUnroll];
    resolve_inplace(a, b, tile + 1, live_next, tile_rows, rows_per_step, row_lane, word_off, col_ok, next);
    // Every load of this tile has returned before any lane stores.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
#pragma unroll
    for (int u = 0; u < kInplaceUnroll; ++u) {
      if (mv[u].src >= 0) {
        *reinterpret_cast<KVC_GLOBAL Chunk*>(kb + mv[u].dst) = kv[u];
        *reinterpret_cast<KVC_GLOBAL Chunk*>(vb + mv[u].dst) = vv[u];
      }
      mv[u] = next[u];
    }
    live = live_next;
  }
}

__global__ void rewrite_tables_kernel(int n_seq, int nb, const int64_t* __restrict__ src_off,
                                      const int64_t* __restrict__ src_ids,
                                      const int64_t* __restrict__ dst_off,
                                      const int64_t* __restrict__ dst_ids,
                                      int64_t* __restrict__ new_tables,
                                      const int64_t* __restrict__ freed_off,
                                      int64_t* __restrict__ freed_ids) {
  const int b = blockIdx.x;
  if (b >= n_seq) return;
  const int64_t* src = src_ids + src_off[b];
  const int64_t n_src = src_off[b + 1] - src_off[b];
  const bool inplace = dst_ids == nullptr;
  const int64_t* dst = inplace ? src : dst_ids + dst_off[b];
  const int64_t n_dst = inplace ? n_src : dst_off[b + 1] - dst_off[b];
  for (int j = threadIdx.x; j < nb; j += blockDim.x)
    new_tables[static_cast<int64_t>(b) * nb + j] = j < n_dst ? dst[j] : -1;
  // Released pages in the reference's order: reversed(source pages not reused).
  const int64_t first_freed = inplace ? (nb < n_src ? nb : n_src) : 0;
  const int64_t n_freed = n_src - first_freed;
  const int64_t room = freed_off[b + 1] - freed_off[b];
  int64_t* out = freed_ids + freed_off[b];
  for (int64_t k = threadIdx.x; k < n_freed && k < room; k += blockDim.x) out[k] = src[n_src - 1 - k];
}

__global__ void token_slots_kernel(const int64_t* __restrict__ block_ids, int64_t n_blocks,
                                   const int64_t* __restrict__ tokens, int64_t n, int block_size,
                                   int64_t* __restrict__ slots) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int64_t t = tokens[i];
  if (t < 0) {
    slots[i] = -1;
    return;
  }
  const int64_t blk = t / block_size;
  slots[i] = blk < n_blocks ? block_ids[blk] * block_size + t % block_size : -1;
}

__global__ void expand_ids_kernel(const int64_t* __restrict__ ids, int64_t n, int k,
                                  int64_t* __restrict__ out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n * k) return;
  out[i] = ids[i / k] * k + i % k;
}

// Slot-addressed row copy in 4-byte words: dst_base[dst_slot] <- src_base[src_slot].
// `gather` reads cache slots into a dense workspace, `!gather` scatters it back.
__global__ void slot_copy_kernel(const char* __restrict__ src, char* __restrict__ dst,
                                 const int64_t* __restrict__ slots, int64_t n_slots,
                                 int64_t num_pages, int64_t page_stride_bytes, int64_t row_bytes,
                                 int gather) {
  const int64_t words = row_bytes / 4;
  const int64_t total = n_slots * words;
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < total;
       e += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t r = e / words, w = e - r * words;
    const int64_t slot = slots[r];
    const int64_t page = slot >> kBlockShift;
    if (slot < 0 || page >= num_pages) continue;
    const int64_t cache_off = page * page_stride_bytes + (slot & (kBlockSize - 1)) * row_bytes + w * 4;
    const int64_t ws_off = r * row_bytes + w * 4;
    if (gather)
      *reinterpret_cast<uint32_t*>(dst + ws_off) = *reinterpret_cast<const uint32_t*>(src + cache_off);
    else
      *reinterpret_cast<uint32_t*>(dst + cache_off) = *reinterpret_cast<const uint32_t*>(src + ws_off);
  }
}

}  // namespace
}  // namespace kvc

using namespace kvc;

extern "C" int kvc_compact(kvc_stream_t stream, int n_layers, const uint64_t* k_layer_ptrs,
                           const uint64_t* v_layer_ptrs, int64_t num_pages, int64_t page_stride,
                           int64_t row_elems, int elem_bytes, int n_seq, const int32_t* seq_lens,
                           const int64_t* src_block_offsets, const int64_t* src_block_ids,
                           const int64_t* dst_block_offsets, const int64_t* dst_block_ids,
                           const int64_t* keep, int64_t keep_stride, int budget, void* workspace,
                           size_t workspace_bytes, int order) {
  if (n_layers <= 0 || n_layers > 65535 || n_seq <= 0 || n_seq > 65535)
    return fail(KVC_EINVAL, "kvc_compact: bad layer or sequence count");
  if (elem_bytes != 2) return fail(KVC_EINVAL, "kvc_compact: elem_bytes must be 2");
  if (order != KVC_COMPACT_LAYER_MAJOR && order != KVC_COMPACT_LAYERS_INTERLEAVED)
    return fail(KVC_EINVAL, "kvc_compact: unknown layer order %d", order);
  if (row_elems <= 0 || budget <= 0 || keep_stride < budget || num_pages <= 0)
    return fail(KVC_EINVAL, "kvc_compact: bad sizes");
  if (page_stride < row_elems * kBlockSize)
    return fail(KVC_EINVAL, "kvc_compact: page stride smaller than a page");
  if (!k_layer_ptrs || !v_layer_ptrs || !seq_lens || !src_block_offsets || !src_block_ids || !keep)
    return fail(KVC_EINVAL, "kvc_compact: null pointer");
  const bool inplace = dst_block_ids == nullptr;
  if (!inplace && !dst_block_offsets)
    return fail(KVC_EINVAL, "kvc_compact: destination offsets missing");

  CompactArgs ca;
  ca.k_ptrs = k_layer_ptrs;
  ca.v_ptrs = v_layer_ptrs;
  ca.n_layers = n_layers;
  ca.n_seq = n_seq;
  ca.num_pages = num_pages;
  ca.page_stride_bytes = page_stride * elem_bytes;
  ca.row_bytes = row_elems * elem_bytes;
  ca.budget = budget;
  ca.seq_lens = seq_lens;
  ca.src_off = src_block_offsets;
  ca.src_ids = src_block_ids;
  ca.dst_off = dst_block_offsets;
  ca.dst_ids = dst_block_ids;
  ca.keep = keep;
  ca.keep_stride = keep_stride;

  // Widest word that divides both the row and the page stride.
  int word = 16;
  while (word > 2 && ((ca.row_bytes % word) != 0 || (ca.page_stride_bytes % word) != 0)) word >>= 1;
  ca.row_chunks = ca.row_bytes / word;

  // Column slice of `threads`-wide workgroups covering `target_chunks` words.
  auto set_slices = [&](int threads, int64_t target_chunks) {
    if (target_chunks > threads) target_chunks = threads;
    int shift = 0;
    while ((1 << shift) < target_chunks) ++shift;
    ca.slice_shift = shift;
    ca.n_slices = static_cast<int>(ceil_div(ca.row_chunks, int64_t(1) << shift));
  };
  // The row-parallel launch's grid, checked before anything is enqueued.
  set_slices(kCopyThreads, ca.row_chunks);
  const int copy_shift = ca.slice_shift, copy_slices = ca.n_slices;
  const int tile_rows = (kCopyThreads >> copy_shift) * kCopyUnroll;
  const int64_t gx = ceil_div(budget, tile_rows) * copy_slices * n_seq;
  if (gx > 0x7fffffff) return fail(KVC_EINVAL, "kvc_compact: grid too large");
  // Planned copy (a workspace for the row offsets and at most kPlanMaxSeqs
  // sequences): its grid is checked here, before anything is enqueued.
  const size_t plan_bytes = static_cast<size_t>(n_seq) * budget * 2 * sizeof(int64_t);
  const bool planned = workspace != nullptr && workspace_bytes >= plan_bytes && n_seq <= kPlanMaxSeqs;
  int plan_shift = 0, plan_slices = 0;
  int64_t per_layer = 0;
  if (planned) {
    if (reinterpret_cast<uintptr_t>(workspace) % 16)
      return fail(KVC_EINVAL, "kvc_compact: workspace must be 16-byte aligned");
    set_slices(kPlanThreads, ca.row_chunks);
    plan_shift = ca.slice_shift;
    plan_slices = ca.n_slices;
    per_layer = ceil_div(budget, kPlanThreads >> plan_shift) * plan_slices * n_seq;
    if (per_layer * n_layers > 0x7fffffff) return fail(KVC_EINVAL, "kvc_compact: grid too large");
  }
  hipStream_t st = as_stream(stream);
  if (inplace) {
    // Hazard rows first, in ordered walks over 256-byte column slices (enough
    // independent workgroups to fill the chip); the safe rows follow below.
    set_slices(kInplaceThreads, 256 / word);
    ca.rows = kRowsHazard;
    dim3 grid(static_cast<unsigned>(ca.n_slices), static_cast<unsigned>(n_seq), static_cast<unsigned>(n_layers));
    switch (word) {
      case 16: compact_inplace_kernel<w128><<<grid, kInplaceThreads, 0, st>>>(ca); break;
      case 8: compact_inplace_kernel<w64><<<grid, kInplaceThreads, 0, st>>>(ca); break;
      case 4: compact_inplace_kernel<uint32_t><<<grid, kInplaceThreads, 0, st>>>(ca); break;
      default: compact_inplace_kernel<uint16_t><<<grid, kInplaceThreads, 0, st>>>(ca); break;
    }
    const int rc = launch_status("kvc_compact");
    if (rc != 0) return rc;
    ca.rows = kRowsSafe;
    ca.dst_off = src_block_offsets;
    ca.dst_ids = src_block_ids;
  } else {
    ca.rows = kRowsAll;
  }
  if (planned) {
    int64_t* plan = static_cast<int64_t*>(workspace);
    ca.slice_shift = plan_shift;
    ca.n_slices = plan_slices;
    const int64_t rows = static_cast<int64_t>(n_seq) * budget;
    compact_plan_kernel<<<static_cast<unsigned>(ceil_div(rows, 256)), 256, 0, st>>>(ca, plan);
    if (int rc = launch_status("kvc_compact(plan)")) return rc;
    const unsigned grid = static_cast<unsigned>(per_layer * n_layers);
    const bool il = order == KVC_COMPACT_LAYERS_INTERLEAVED;
    // Buffer offsets are 32-bit: every row of a layer must lie below 4 GiB of
    // its buffer's base.
    const bool sc1_stores = !il && static_cast<uint64_t>(num_pages) * static_cast<uint64_t>(ca.page_stride_bytes) <= 0xFFFFFFFFull;
    switch (word) {
      case 16:
        if (sc1_stores)
          compact_layer_kernel<w128, true><<<grid, kPlanThreads, 0, st>>>(ca, plan, per_layer, il);
        else
          compact_layer_kernel<w128><<<grid, kPlanThreads, 0, st>>>(ca, plan, per_layer, il);
        break;
      case 8: compact_layer_kernel<w64><<<grid, kPlanThreads, 0, st>>>(ca, plan, per_layer, il); break;
      case 4: compact_layer_kernel<uint32_t><<<grid, kPlanThreads, 0, st>>>(ca, plan, per_layer, il); break;
      default: compact_layer_kernel<uint16_t><<<grid, kPlanThreads, 0, st>>>(ca, plan, per_layer, il); break;
    }
    return launch_status("kvc_compact");
  }
  // Whole rows (up to the workgroup width) per workgroup.
  ca.slice_shift = copy_shift;
  ca.n_slices = copy_slices;
  dim3 grid(static_cast<unsigned>(gx));
  switch (word) {
    case 16: compact_private_kernel<w128><<<grid, kCopyThreads, 0, st>>>(ca); break;
    case 8: compact_private_kernel<w64><<<grid, kCopyThreads, 0, st>>>(ca); break;
    case 4: compact_private_kernel<uint32_t><<<grid, kCopyThreads, 0, st>>>(ca); break;
    default: compact_private_kernel<uint16_t><<<grid, kCopyThreads, 0, st>>>(ca); break;
  }
  return launch_status("kvc_compact");
}

extern "C" size_t kvc_compact_workspace_bytes(int n_seq, int budget) {
  if (n_seq <= 0 || budget <= 0) return 0;
  return (static_cast<size_t>(n_seq) * budget * 2 * sizeof(int64_t) + 255) / 256 * 256;
}

extern "C" int kvc_rewrite_block_tables(kvc_stream_t stream, int n_seq, int budget,
                                        const int64_t* src_block_offsets,
                                        const int64_t* src_block_ids,
                                        const int64_t* dst_block_offsets,
                                        const int64_t* dst_block_ids, int64_t* new_tables,
                                        const int64_t* freed_offsets, int64_t* freed_ids) {
  if (n_seq <= 0 || budget <= 0) return fail(KVC_EINVAL, "kvc_rewrite_block_tables: bad sizes");
  if (!src_block_offsets || !src_block_ids || !new_tables || !freed_offsets || !freed_ids)
    return fail(KVC_EINVAL, "kvc_rewrite_block_tables: null pointer");
  if (dst_block_ids && !dst_block_offsets)
    return fail(KVC_EINVAL, "kvc_rewrite_block_tables: destination offsets missing");
  const int nb = static_cast<int>(ceil_div(budget, kBlockSize));
  rewrite_tables_kernel<<<n_seq, 256, 0, as_stream(stream)>>>(
      n_seq, nb, src_block_offsets, src_block_ids, dst_block_offsets, dst_block_ids, new_tables,
      freed_offsets, freed_ids);
  return launch_status("kvc_rewrite_block_tables");
}

extern "C" int kvc_token_slots(kvc_stream_t stream, const int64_t* block_ids, int64_t n_blocks,
                               const int64_t* token_indices, int64_t n_tokens, int block_size,
                               int64_t* slots) {
  if (n_tokens < 0 || n_blocks < 0 || block_size <= 0)
    return fail(KVC_EINVAL, "kvc_token_slots: bad sizes");
  if (n_tokens == 0) return 0;
  if (!block_ids || !token_indices || !slots) return fail(KVC_EINVAL, "kvc_token_slots: null pointer");
  token_slots_kernel<<<static_cast<unsigned>(ceil_div(n_tokens, 256)), 256, 0, as_stream(stream)>>>(
      block_ids, n_blocks, token_indices, n_tokens, block_size, slots);
  return launch_status("kvc_token_slots");
}

extern "C" int kvc_expand_block_ids(kvc_stream_t stream, const int64_t* ids, int64_t n_ids, int k,
                                    int64_t* out) {
  if (n_ids < 0 || k <= 0) return fail(KVC_EINVAL, "kvc_expand_block_ids: bad sizes");
  if (n_ids == 0) return 0;
  if (!ids || !out) return fail(KVC_EINVAL, "kvc_expand_block_ids: null pointer");
  const int64_t total = n_ids * k;
  expand_ids_kernel<<<static_cast<unsigned>(ceil_div(total, 256)), 256, 0, as_stream(stream)>>>(
      ids, n_ids, k, out);
  return launch_status("kvc_expand_block_ids");
}

extern "C" int kvc_materialize_slots(kvc_stream_t stream, void* k_cache, void* v_cache,
                                     int64_t num_pages, int64_t page_stride, int64_t row_elems,
                                     int elem_bytes, const int64_t* src_slots,
                                     const int64_t* dst_slots, int64_t n_slots, void* k_ws,
                                     void* v_ws) {
  if (elem_bytes != 2 || row_elems <= 0 || num_pages <= 0 || n_slots < 0)
    return fail(KVC_EINVAL, "kvc_materialize_slots: bad sizes");
  if (page_stride < row_elems * kBlockSize)
    return fail(KVC_EINVAL, "kvc_materialize_slots: page stride smaller than a page");
  const int64_t row_bytes = row_elems * elem_bytes;
  const int64_t ps_bytes = page_stride * elem_bytes;
  if (row_bytes % 4 != 0 || ps_bytes % 4 != 0)
    return fail(KVC_EINVAL, "kvc_materialize_slots: rows and pages must be 4-byte multiples");
  if (n_slots == 0) return 0;
  if (!k_cache || !v_cache || !src_slots || !dst_slots || !k_ws || !v_ws)
    return fail(KVC_EINVAL, "kvc_materialize_slots: null pointer");
  hipStream_t st = as_stream(stream);
  const int64_t total = n_slots * (row_bytes / 4);
  const unsigned blocks = static_cast<unsigned>(ceil_div(total, 256) < 65536 ? ceil_div(total, 256) : 65536);
  slot_copy_kernel<<<blocks, 256, 0, st>>>(static_cast<const char*>(k_cache),
                                           static_cast<char*>(k_ws), src_slots, n_slots, num_pages,
                                           ps_bytes, row_bytes, 1);
  slot_copy_kernel<<<blocks, 256, 0, st>>>(static_cast<const char*>(v_cache),
                                           static_cast<char*>(v_ws), src_slots, n_slots, num_pages,
                                           ps_bytes, row_bytes, 1);
  slot_copy_kernel<<<blocks, 256, 0, st>>>(static_cast<const char*>(k_ws),
                                           static_cast<char*>(k_cache), dst_slots, n_slots,
                                           num_pages, ps_bytes, row_bytes, 0);
  slot_copy_kernel<<<blocks, 256, 0, st>>>(static_cast<const char*>(v_ws),
                                           static_cast<char*>(v_cache), dst_slots, n_slots,
                                           num_pages, ps_bytes, row_bytes, 0);
  return launch_status("kvc_materialize_slots");
}
