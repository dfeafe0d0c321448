// CSR construction on the device: per-key counts, exclusive prefix sum,
// stable grouping order and the GIE grouping step.
//
// Restates python/kernels/segment.py:46-71 (segment_offsets = [0] ++
// cumsum(bincount(keys)), group_by_source = stable argsort + offsets) as
// device passes:
//   1. fill      counts[N] = 0, flags = 0
//   2. histogram counts[k] += 1 per key (64-bit integer atomics: integer
//                addition commutes, so the counts are exact whatever the
//                interleaving), range and sortedness flags
//   3. scan      offsets[n + 1] = sum_{m <= n} counts[m], in three passes
//                (tile totals, scan of the totals, tile scans)
//   4. order     stable radix sort of the keys (sort.hip), only when needed.
// The integer results are bit-exact.  Functions that report an index-range
// error read the flags back and therefore synchronise the stream.
#include "common.h"

namespace dpa4k {

// Stable argsort of int64 keys known to lie in [0, n_nodes) (sort.hip).
size_t stable_order_workspace(int64_t n_edges, int64_t n_nodes);
int stable_order(const int64_t* keys, int64_t n_edges, int64_t n_nodes, int64_t* order,
                 void* workspace, size_t workspace_bytes, hipStream_t stream);

namespace {

constexpr int kScanThreads = 256;
constexpr int kScanItems = 16;
constexpr int64_t kScanTile = kScanThreads * kScanItems;

enum : int32_t { kFlagOutOfRange = 1, kFlagUnsorted = 2, kFlagSlotRange = 4, kFlagSlotShared = 8 };

__global__ __launch_bounds__(256) void fill_i64_kernel(int64_t* __restrict__ data, int64_t n,
                                                       int32_t* __restrict__ flags) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
    data[i] = 0;
  if (blockIdx.x == 0 && threadIdx.x == 0 && flags != nullptr) *flags = 0;
}

__global__ __launch_bounds__(256) void histogram_kernel(const int64_t* __restrict__ keys,
                                                        int64_t n_edges, int64_t n_nodes,
                                                        int64_t* __restrict__ counts,
                                                        int32_t* __restrict__ flags) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  int32_t local = 0;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n_edges;
       i += stride) {
    const int64_t key = keys[i];
    if (static_cast<uint64_t>(key) >= static_cast<uint64_t>(n_nodes)) {
      local |= kFlagOutOfRange;
    } else {
      atomicAdd(reinterpret_cast<unsigned long long*>(counts + key), 1ull);
    }
    if (i + 1 < n_edges && keys[i + 1] < key) local |= kFlagUnsorted;
  }
  if (local != 0) atomicOr(flags, local);
}

// Block-wide inclusive scan of one int64 per thread (Hillis-Steele in LDS).
__device__ int64_t block_inclusive_scan(int64_t value, int64_t* lds) {
  const int t = threadIdx.x;
  lds[t] = value;
  __syncthreads();
  for (int offset = 1; offset < kScanThreads; offset <<= 1) {
    const int64_t add = t >= offset ? lds[t - offset] : 0;
    __syncthreads();
    lds[t] += add;
    __syncthreads();
  }
  const int64_t result = lds[t];
  __syncthreads();
  return result;
}

__global__ __launch_bounds__(kScanThreads) void tile_total_kernel(const int64_t* __restrict__ counts,
                                                                  int64_t n, int64_t* __restrict__ totals) {
  __shared__ int64_t lds[kScanThreads];
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kScanTile;
  int64_t sum = 0;
  for (int i = 0; i < kScanItems; ++i) {
    const int64_t index = base + static_cast<int64_t>(i) * kScanThreads + threadIdx.x;
    if (index < n) sum += counts[index];
  }
  const int64_t inclusive = block_inclusive_scan(sum, lds);
  if (threadIdx.x == kScanThreads - 1) totals[blockIdx.x] = inclusive;
}

// Exclusive scan of the tile totals in place, by one block; each thread owns
// a contiguous run of ceil(n / 256) totals.
__global__ __launch_bounds__(kScanThreads) void scan_totals_kernel(int64_t* __restrict__ totals,
                                                                   int64_t n) {
  __shared__ int64_t lds[kScanThreads];
  const int64_t per_thread = (n + kScanThreads - 1) / kScanThreads;
  const int64_t begin = static_cast<int64_t>(threadIdx.x) * per_thread;
  const int64_t end = begin + per_thread < n ? begin + per_thread : n;
  int64_t sum = 0;
  for (int64_t i = begin; i < end; ++i) sum += totals[i];
  const int64_t inclusive = block_inclusive_scan(sum, lds);
  int64_t running = inclusive - sum;
  for (int64_t i = begin; i < end; ++i) {
    const int64_t value = totals[i];
    totals[i] = running;
    running += value;
  }
}

// offsets[i + 1] = prefix(tile) + inclusive scan of counts inside the tile.
// Thread t owns the kScanItems consecutive counts [base + t*items, ...).
__global__ __launch_bounds__(kScanThreads) void tile_scan_kernel(const int64_t* __restrict__ counts,
                                                                 int64_t n,
                                                                 const int64_t* __restrict__ tile_prefix,
                                                                 int64_t* __restrict__ offsets) {
  __shared__ int64_t lds[kScanThreads];
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kScanTile +
                       static_cast<int64_t>(threadIdx.x) * kScanItems;
  int64_t values[kScanItems];
  int64_t sum = 0;
#pragma unroll
  for (int i = 0; i < kScanItems; ++i) {
    const int64_t index = base + i;
    values[i] = index < n ? counts[index] : 0;
    sum += values[i];
  }
  const int64_t inclusive = block_inclusive_scan(sum, lds);
  int64_t running = tile_prefix[blockIdx.x] + inclusive - sum;
#pragma unroll
  for (int i = 0; i < kScanItems; ++i) {
    const int64_t index = base + i;
    running += values[i];
    if (index < n) offsets[index + 1] = running;
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) offsets[0] = 0;
}

// Range and sharing checks of the GIE radial slots (one small block).
__global__ __launch_bounds__(64) void slot_check_kernel(const int64_t* __restrict__ radial_slot,
                                                        int64_t n_rows, int64_t n_radial,
                                                        int32_t* __restrict__ flags) {
  int32_t local = 0;
  for (int64_t r = threadIdx.x; r < n_rows; r += blockDim.x) {
    const int64_t slot = radial_slot[r];
    if (static_cast<uint64_t>(slot) >= static_cast<uint64_t>(n_radial)) local |= kFlagSlotRange;
    for (int64_t other = r + 1; other < n_rows; ++other)
      if (radial_slot[other] == slot) local |= kFlagSlotShared;
  }
  if (local != 0) atomicOr(flags, local);
}

struct OffsetsScratch {
  int64_t* counts;
  int64_t* totals;
  int32_t* flags;
};

int64_t tiles_for(int64_t n_nodes) { return (n_nodes + kScanTile - 1) / kScanTile; }

size_t offsets_scratch_bytes(int64_t n_nodes) {
  return round_up_256(static_cast<size_t>(n_nodes) * 8) +
         round_up_256(static_cast<size_t>(tiles_for(n_nodes)) * 8) + 256;
}

bool carve_offsets(Carver& carver, int64_t n_nodes, OffsetsScratch& out) {
  out.counts = carver.take<int64_t>(static_cast<size_t>(n_nodes));
  out.totals = carver.take<int64_t>(static_cast<size_t>(tiles_for(n_nodes)));
  out.flags = carver.take<int32_t>(1);
  return out.counts && out.totals && out.flags;
}

unsigned int grid_stride_blocks(int64_t items) {
  const int64_t wanted = (items + 255) / 256;
  return static_cast<unsigned int>(wanted < 1 ? 1 : (wanted > 8192 ? 8192 : wanted));
}

// Enqueues fill + histogram + scan.  No synchronisation.
int enqueue_offsets(const int64_t* keys, int64_t n_edges, int64_t n_nodes, int64_t* offsets,
                    const OffsetsScratch& scratch, hipStream_t stream) {
  fill_i64_kernel<<<grid_stride_blocks(n_nodes), 256, 0, stream>>>(scratch.counts, n_nodes,
                                                                    scratch.flags);
  if (int s = launched("fill_i64_kernel")) return s;
  if (n_edges > 0) {
    histogram_kernel<<<grid_stride_blocks(n_edges), 256, 0, stream>>>(keys, n_edges, n_nodes,
                                                                      scratch.counts, scratch.flags);
    if (int s = launched("histogram_kernel")) return s;
  }
  const int64_t tiles = tiles_for(n_nodes);
  tile_total_kernel<<<static_cast<unsigned int>(tiles), kScanThreads, 0, stream>>>(
      scratch.counts, n_nodes, scratch.totals);
  if (int s = launched("tile_total_kernel")) return s;
  scan_totals_kernel<<<1, kScanThreads, 0, stream>>>(scratch.totals, tiles);
  if (int s = launched("scan_totals_kernel")) return s;
  tile_scan_kernel<<<static_cast<unsigned int>(tiles), kScanThreads, 0, stream>>>(
      scratch.counts, n_nodes, scratch.totals, offsets);
  return launched("tile_scan_kernel");
}

int read_flags(const int32_t* flags, int32_t& host, hipStream_t stream) {
  if (int s = hip_status(hipMemcpyAsync(&host, flags, sizeof(int32_t), hipMemcpyDeviceToHost, stream),
                         "hipMemcpyAsync(flags)"))
    return s;
  return hip_status(hipStreamSynchronize(stream), "hipStreamSynchronize");
}

int check_sizes(int64_t n_edges, int64_t n_nodes, const char* what) {
  if (n_edges < 0) return fail(DPA4K_EINVAL, "%s: negative edge count", what);
  if (n_nodes <= 0) return fail(DPA4K_EINVAL, "%s require a positive node count", what);
  if (tiles_for(n_nodes) > kMaxGrid) return fail(DPA4K_EINVAL, "%s: node count too large", what);
  return DPA4K_OK;
}

}  // namespace
}  // namespace dpa4k

using namespace dpa4k;

extern "C" size_t dpa4k_segment_offsets_workspace_size(int64_t n_edges, int64_t n_nodes) {
  (void)n_edges;
  return n_nodes > 0 ? offsets_scratch_bytes(n_nodes) : 0;
}

extern "C" int dpa4k_segment_offsets(const int64_t* keys, int64_t n_edges, int64_t n_nodes,
                                     int64_t* offsets, void* workspace, size_t workspace_bytes,
                                     dpa4k_stream_t stream_handle) {
  clear_error();
  if (int s = check_sizes(n_edges, n_nodes, "segment offsets")) return s;
  if (offsets == nullptr || (n_edges > 0 && keys == nullptr))
    return fail(DPA4K_EINVAL, "segment offsets: null pointer");
  Carver carver{static_cast<char*>(workspace), workspace_bytes};
  OffsetsScratch scratch{};
  if (workspace == nullptr || !carve_offsets(carver, n_nodes, scratch))
    return fail(DPA4K_EWORKSPACE, "segment offsets: workspace of %zu bytes is smaller than %zu",
                workspace_bytes, offsets_scratch_bytes(n_nodes));
  hipStream_t stream = as_stream(stream_handle);
  if (int s = enqueue_offsets(keys, n_edges, n_nodes, offsets, scratch, stream)) return s;
  int32_t flags = 0;
  if (int s = read_flags(scratch.flags, flags, stream)) return s;
  if (flags & kFlagOutOfRange)
    return fail(DPA4K_EINVAL, "destination values must be within the node range");
  return DPA4K_OK;
}

extern "C" size_t dpa4k_group_by_key_workspace_size(int64_t n_edges, int64_t n_nodes) {
  if (n_nodes <= 0) return 0;
  const size_t a = offsets_scratch_bytes(n_nodes);
  const size_t b = stable_order_workspace(n_edges, n_nodes);
  return a > b ? a : b;
}

extern "C" int dpa4k_group_by_key(const int64_t* keys, int64_t n_edges, int64_t n_nodes,
                                  int64_t* order, int64_t* offsets, void* workspace,
                                  size_t workspace_bytes, dpa4k_stream_t stream_handle) {
  clear_error();
  if (int s = check_sizes(n_edges, n_nodes, "group_by_source")) return s;
  if (offsets == nullptr || (n_edges > 0 && (keys == nullptr || order == nullptr)))
    return fail(DPA4K_EINVAL, "group_by_source: null pointer");
  const size_t needed = dpa4k_group_by_key_workspace_size(n_edges, n_nodes);
  if (workspace == nullptr || workspace_bytes < needed)
    return fail(DPA4K_EWORKSPACE, "group_by_source: workspace of %zu bytes is smaller than %zu",
                workspace_bytes, needed);
  hipStream_t stream = as_stream(stream_handle);
  Carver carver{static_cast<char*>(workspace), workspace_bytes};
  OffsetsScratch scratch{};
  carve_offsets(carver, n_nodes, scratch);
  if (int s = enqueue_offsets(keys, n_edges, n_nodes, offsets, scratch, stream)) return s;
  int32_t flags = 0;
  if (int s = read_flags(scratch.flags, flags, stream)) return s;
  if (flags & kFlagOutOfRange)
    return fail(DPA4K_EINVAL, "source values must be within the node range");
  if (n_edges == 0) return DPA4K_OK;
  // The offsets scratch is dead once the flags are read: the sort reuses the
  // whole workspace.
  return stable_order(keys, n_edges, n_nodes, order, workspace, workspace_bytes, stream);
}

extern "C" size_t dpa4k_gie_group_workspace_size(int64_t n_edges, int64_t n_nodes) {
  return dpa4k_group_by_key_workspace_size(n_edges, n_nodes);
}

extern "C" int dpa4k_gie_group(const int64_t* dst, const int64_t* radial_slot, int64_t n_edges,
                               int64_t n_nodes, int64_t n_rows, int64_t n_radial, int64_t* offsets,
                               int64_t* order, int32_t* host_info, void* workspace,
                               size_t workspace_bytes, dpa4k_stream_t stream_handle) {
  clear_error();
  if (int s = check_sizes(n_edges, n_nodes, "GIE grouping")) return s;
  if (n_rows < 0 || n_radial < 0) return fail(DPA4K_EINVAL, "GIE grouping: negative sizes");
  if (offsets == nullptr || (n_edges > 0 && dst == nullptr) ||
      (n_rows > 0 && radial_slot == nullptr))
    return fail(DPA4K_EINVAL, "GIE grouping: null pointer");
  const size_t needed = dpa4k_gie_group_workspace_size(n_edges, n_nodes);
  if (workspace == nullptr || workspace_bytes < needed)
    return fail(DPA4K_EWORKSPACE, "GIE grouping: workspace of %zu bytes is smaller than %zu",
                workspace_bytes, needed);
  hipStream_t stream = as_stream(stream_handle);
  Carver carver{static_cast<char*>(workspace), workspace_bytes};
  OffsetsScratch scratch{};
  carve_offsets(carver, n_nodes, scratch);
  if (int s = enqueue_offsets(dst, n_edges, n_nodes, offsets, scratch, stream)) return s;
  if (n_rows > 0) {
    slot_check_kernel<<<1, 64, 0, stream>>>(radial_slot, n_rows, n_radial, scratch.flags);
    if (int s = launched("slot_check_kernel")) return s;
  }
  int32_t flags = 0;
  if (int s = read_flags(scratch.flags, flags, stream)) return s;
  if (flags & kFlagOutOfRange) return fail(DPA4K_EINVAL, "GIE dst values must be within the node range");
  if (flags & kFlagSlotRange)
    return fail(DPA4K_EINVAL, "GIE radial_slot values must be within the radial range");
  int32_t info = 0;
  if (!(flags & kFlagUnsorted)) info |= 1;
  if (!(flags & kFlagSlotShared)) info |= 2;
  if (host_info != nullptr) *host_info = info;
  if ((info & 1) || n_edges == 0) return DPA4K_OK;
  if (order == nullptr) return fail(DPA4K_EINVAL, "GIE grouping: unsorted dst needs an order buffer");
  return stable_order(dst, n_edges, n_nodes, order, workspace, workspace_bytes, stream);
}
