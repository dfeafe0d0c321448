// CSR construction on the device: offsets, stable grouping order and the GIE
// grouping step.
//
// Restates python/kernels/segment.py:46-71 (segment_offsets = [0] ++
// cumsum(bincount(keys)), group_by_source = stable argsort + offsets) without
// a histogram:
//   1. check     one streaming pass over the keys: range and sortedness
//                flags (at most one integer OR per workgroup); the host
//                reads them back, as the reference's dst.min()/dst.max()
//                check does, and raises on out-of-range keys;
//   2. sort      keys that are not already non-decreasing are sorted by a
//                stable LSD radix sort (sort.hip), alone or with their
//                positions (the grouping order);
//   3. bounds    offsets from the sorted keys: position e writes
//                offsets[k] = e for every k in (key[e-1], key[e]] (with
//                key[-1] = -1 and key[E] = N), so every entry is written
//                exactly once, by the first edge of its segment.
// Sorted keys (DeepMD's usual layout) need only passes 1 and 3.  Integer
// results are bit-exact; nothing depends on scheduling.
#include "common.h"

namespace dpa4k {

// Stable sort of keys in [0, n_nodes) (sort.hip).
size_t sort_workspace(int64_t n_edges, int64_t n_nodes);
int sort_keys(const int64_t* keys, int64_t n_edges, int64_t n_nodes, uint32_t* sorted_keys, int64_t* order,
              void* workspace, size_t workspace_bytes, hipStream_t stream);

namespace {

enum : int32_t { kFlagOutOfRange = 1, kFlagUnsorted = 2, kFlagSlotRange = 4, kFlagSlotShared = 8 };

unsigned int grid_stride_blocks(int64_t items, int64_t cap = 8192) {
  const int64_t wanted = (items + 255) / 256;
  return static_cast<unsigned int>(wanted < 1 ? 1 : (wanted > cap ? cap : wanted));
}

__global__ __launch_bounds__(64) void clear_flags_kernel(int32_t* __restrict__ flags) {
  if (threadIdx.x == 0) *flags = 0;
}

__global__ __launch_bounds__(256) void check_keys_kernel(const int64_t* __restrict__ keys, int64_t n_edges,
                                                         int64_t n_nodes, int32_t* __restrict__ flags) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  int32_t local = 0;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n_edges; i += stride) {
    const int64_t key = keys[i];
    if (static_cast<uint64_t>(key) >= static_cast<uint64_t>(n_nodes)) local |= kFlagOutOfRange;
    if (i + 1 < n_edges && keys[i + 1] < key) local |= kFlagUnsorted;
  }
  // one OR per workgroup, skipped when another workgroup already set the bits
  // (many workgroups hitting one word would serialise in the L2)
  const int32_t found = (__syncthreads_or(local & kFlagOutOfRange) ? kFlagOutOfRange : 0) |
                        (__syncthreads_or(local & kFlagUnsorted) ? kFlagUnsorted : 0);
  if (threadIdx.x == 0 && found != 0 && (__atomic_load_n(flags, __ATOMIC_RELAXED) & found) != found)
    atomicOr(flags, found);
}

// offsets[k] = first position e with key[e] >= k, for k in [0, n_nodes], of
// non-decreasing keys in [0, n_nodes).
template <typename K>
__global__ __launch_bounds__(256) void offsets_from_sorted_kernel(const K* __restrict__ keys, int64_t n_edges,
                                                                  int64_t n_nodes, int64_t* __restrict__ offsets) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e <= n_edges; e += stride) {
    const int64_t previous = e > 0 ? static_cast<int64_t>(keys[e - 1]) : -1;
    const int64_t current = e < n_edges ? static_cast<int64_t>(keys[e]) : n_nodes;
    for (int64_t k = previous + 1; k <= current && k <= n_nodes; ++k) offsets[k] = e;
  }
}

__global__ __launch_bounds__(256) void iota_kernel(int64_t* __restrict__ order, int64_t n) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) order[i] = i;
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

// Workspace: the flags word, the sorted 32-bit keys, the sort's scratch.
struct Scratch {
  int32_t* flags = nullptr;
  uint32_t* sorted = nullptr;
  void* sort = nullptr;
  size_t sort_bytes = 0;
};

size_t scratch_bytes(int64_t n_edges, int64_t n_nodes) {
  const size_t edges = static_cast<size_t>(n_edges > 0 ? n_edges : 1);
  const size_t sort = sort_workspace(n_edges, n_nodes);
  return 256 + round_up_256(edges * sizeof(uint32_t)) + round_up_256(sort > 0 ? sort : 1);
}

bool carve(void* workspace, size_t bytes, int64_t n_edges, int64_t n_nodes, Scratch& out) {
  if (workspace == nullptr || bytes < scratch_bytes(n_edges, n_nodes)) return false;
  Carver carver{static_cast<char*>(workspace), bytes};
  out.flags = carver.take<int32_t>(1);
  out.sorted = carver.take<uint32_t>(static_cast<size_t>(n_edges > 0 ? n_edges : 1));
  out.sort_bytes = sort_workspace(n_edges, n_nodes);
  out.sort = carver.take<char>(out.sort_bytes > 0 ? out.sort_bytes : 1);
  return out.flags && out.sorted && out.sort;
}

// Pass 1 (+ optional slot checks), then the flags are read back.  Synchronises.
int check_keys(const int64_t* keys, int64_t n_edges, int64_t n_nodes, const int64_t* radial_slot, int64_t n_rows,
               int64_t n_radial, const Scratch& scratch, int32_t& flags, hipStream_t stream) {
  clear_flags_kernel<<<1, 64, 0, stream>>>(scratch.flags);
  if (int s = launched("clear_flags_kernel")) return s;
  if (n_edges > 0) {
    check_keys_kernel<<<grid_stride_blocks(n_edges, 2048), 256, 0, stream>>>(keys, n_edges, n_nodes,
                                                                             scratch.flags);
    if (int s = launched("check_keys_kernel")) return s;
  }
  if (n_rows > 0) {
    slot_check_kernel<<<1, 64, 0, stream>>>(radial_slot, n_rows, n_radial, scratch.flags);
    if (int s = launched("slot_check_kernel")) return s;
  }
  int32_t host = 0;
  if (int s = hip_status(hipMemcpyAsync(&host, scratch.flags, sizeof(int32_t), hipMemcpyDeviceToHost, stream),
                         "hipMemcpyAsync(flags)"))
    return s;
  if (int s = hip_status(hipStreamSynchronize(stream), "hipStreamSynchronize")) return s;
  flags = host;
  return DPA4K_OK;
}

// Passes 2 and 3 for checked keys: offsets always, the order when `order` is
// given (the identity for sorted keys).
int build(const int64_t* keys, int64_t n_edges, int64_t n_nodes, bool sorted, int64_t* offsets, int64_t* order,
          const Scratch& scratch, hipStream_t stream) {
  const unsigned int blocks = grid_stride_blocks(n_edges + 1);
  if (sorted || n_edges == 0) {
    if (order != nullptr && n_edges > 0) {
      iota_kernel<<<grid_stride_blocks(n_edges), 256, 0, stream>>>(order, n_edges);
      if (int s = launched("iota_kernel")) return s;
    }
    offsets_from_sorted_kernel<int64_t><<<blocks, 256, 0, stream>>>(keys, n_edges, n_nodes, offsets);
    return launched("offsets_from_sorted_kernel");
  }
  if (int s = sort_keys(keys, n_edges, n_nodes, scratch.sorted, order, scratch.sort, scratch.sort_bytes, stream))
    return s;
  offsets_from_sorted_kernel<uint32_t><<<blocks, 256, 0, stream>>>(scratch.sorted, n_edges, n_nodes, offsets);
  return launched("offsets_from_sorted_kernel");
}

int check_sizes(int64_t n_edges, int64_t n_nodes, const char* what) {
  if (n_edges < 0) return fail(DPA4K_EINVAL, "%s: negative edge count", what);
  if (n_nodes <= 0) return fail(DPA4K_EINVAL, "%s require a positive node count", what);
  if (n_nodes > (int64_t(1) << 32)) return fail(DPA4K_EINVAL, "%s supports at most 2^32 nodes", what);
  return DPA4K_OK;
}

}  // namespace
}  // namespace dpa4k

using namespace dpa4k;

extern "C" size_t dpa4k_segment_offsets_workspace_size(int64_t n_edges, int64_t n_nodes) {
  return n_nodes > 0 ? scratch_bytes(n_edges, n_nodes) : 0;
}

extern "C" int dpa4k_segment_offsets(const int64_t* keys, int64_t n_edges, int64_t n_nodes, int64_t* offsets,
                                     void* workspace, size_t workspace_bytes, dpa4k_stream_t stream_handle) {
  clear_error();
  if (int s = check_sizes(n_edges, n_nodes, "segment offsets")) return s;
  if (offsets == nullptr || (n_edges > 0 && keys == nullptr)) return fail(DPA4K_EINVAL, "segment offsets: null pointer");
  Scratch scratch;
  if (!carve(workspace, workspace_bytes, n_edges, n_nodes, scratch))
    return fail(DPA4K_EWORKSPACE, "segment offsets: workspace of %zu bytes is smaller than %zu", workspace_bytes,
                scratch_bytes(n_edges, n_nodes));
  hipStream_t stream = as_stream(stream_handle);
  int32_t flags = 0;
  if (int s = check_keys(keys, n_edges, n_nodes, nullptr, 0, 0, scratch, flags, stream)) return s;
  if (flags & kFlagOutOfRange) return fail(DPA4K_EINVAL, "destination values must be within the node range");
  return build(keys, n_edges, n_nodes, !(flags & kFlagUnsorted), offsets, nullptr, scratch, stream);
}

extern "C" size_t dpa4k_group_by_key_workspace_size(int64_t n_edges, int64_t n_nodes) {
  return n_nodes > 0 ? scratch_bytes(n_edges, n_nodes) : 0;
}

extern "C" int dpa4k_group_by_key(const int64_t* keys, int64_t n_edges, int64_t n_nodes, int64_t* order,
                                  int64_t* offsets, void* workspace, size_t workspace_bytes,
                                  dpa4k_stream_t stream_handle) {
  clear_error();
  if (int s = check_sizes(n_edges, n_nodes, "group_by_source")) return s;
  if (offsets == nullptr || (n_edges > 0 && (keys == nullptr || order == nullptr)))
    return fail(DPA4K_EINVAL, "group_by_source: null pointer");
  Scratch scratch;
  if (!carve(workspace, workspace_bytes, n_edges, n_nodes, scratch))
    return fail(DPA4K_EWORKSPACE, "group_by_source: workspace of %zu bytes is smaller than %zu", workspace_bytes,
                scratch_bytes(n_edges, n_nodes));
  hipStream_t stream = as_stream(stream_handle);
  int32_t flags = 0;
  if (int s = check_keys(keys, n_edges, n_nodes, nullptr, 0, 0, scratch, flags, stream)) return s;
  if (flags & kFlagOutOfRange) return fail(DPA4K_EINVAL, "source values must be within the node range");
  return build(keys, n_edges, n_nodes, !(flags & kFlagUnsorted), offsets, order, scratch, stream);
}

extern "C" size_t dpa4k_gie_group_workspace_size(int64_t n_edges, int64_t n_nodes) {
  return dpa4k_group_by_key_workspace_size(n_edges, n_nodes);
}

extern "C" int dpa4k_gie_group(const int64_t* dst, const int64_t* radial_slot, int64_t n_edges, int64_t n_nodes,
                               int64_t n_rows, int64_t n_radial, int64_t* offsets, int64_t* order,
                               int32_t* host_info, void* workspace, size_t workspace_bytes,
                               dpa4k_stream_t stream_handle) {
  clear_error();
  if (int s = check_sizes(n_edges, n_nodes, "GIE grouping")) return s;
  if (n_rows < 0 || n_radial < 0) return fail(DPA4K_EINVAL, "GIE grouping: negative sizes");
  if (offsets == nullptr || (n_edges > 0 && dst == nullptr) || (n_rows > 0 && radial_slot == nullptr))
    return fail(DPA4K_EINVAL, "GIE grouping: null pointer");
  Scratch scratch;
  if (!carve(workspace, workspace_bytes, n_edges, n_nodes, scratch))
    return fail(DPA4K_EWORKSPACE, "GIE grouping: workspace of %zu bytes is smaller than %zu", workspace_bytes,
                scratch_bytes(n_edges, n_nodes));
  hipStream_t stream = as_stream(stream_handle);
  int32_t flags = 0;
  if (int s = check_keys(dst, n_edges, n_nodes, radial_slot, n_rows, n_radial, scratch, flags, stream)) return s;
  if (flags & kFlagOutOfRange) return fail(DPA4K_EINVAL, "GIE dst values must be within the node range");
  if (flags & kFlagSlotRange) return fail(DPA4K_EINVAL, "GIE radial_slot values must be within the radial range");
  const bool sorted = !(flags & kFlagUnsorted);
  const int32_t info = (sorted ? 1 : 0) | ((flags & kFlagSlotShared) ? 0 : 2);
  if (host_info != nullptr) *host_info = info;
  if (!sorted && n_edges > 0 && order == nullptr)
    return fail(DPA4K_EINVAL, "GIE grouping: unsorted dst needs an order buffer");
  return build(dst, n_edges, n_nodes, sorted, offsets, sorted ? nullptr : order, scratch, stream);
}
