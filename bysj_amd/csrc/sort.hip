// Stable argsort of bounded int64 keys (the grouping order of
// python/kernels/segment.py:70, `torch.argsort(src, stable=True)`).
//
// The keys are narrowed to uint32 and sorted (alone, or together with the
// identity permutation) by rocPRIM's LSD radix sort, which is stable; only
// the ceil(log2(n_nodes)) low bits are sorted.  A stable order of a key list
// is unique, so the result is bit-exact and independent of scheduling.  All
// scratch memory comes from the caller's workspace.
#include <rocprim/device/device_radix_sort.hpp>
#include <rocprim/iterator/counting_iterator.hpp>

#include "common.h"

namespace dpa4k {
namespace {

__global__ __launch_bounds__(256) void narrow_keys_kernel(const int64_t* __restrict__ keys,
                                                          int64_t n, uint32_t* __restrict__ out) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
    out[i] = static_cast<uint32_t>(keys[i]);
}

unsigned int key_bits(int64_t n_nodes) {
  unsigned int bits = 1;
  while (bits < 32 && (int64_t(1) << bits) < n_nodes) ++bits;
  return bits;
}

size_t rocprim_bytes(int64_t n_edges, int64_t n_nodes, bool with_order) {
  size_t bytes = 0;
  uint32_t* keys = nullptr;
  int64_t* values = nullptr;
  rocprim::counting_iterator<int64_t> identity(0);
  const hipError_t status =
      with_order ? rocprim::radix_sort_pairs(nullptr, bytes, keys, keys, identity, values,
                                             static_cast<size_t>(n_edges), 0, key_bits(n_nodes))
                 : rocprim::radix_sort_keys(nullptr, bytes, keys, keys, static_cast<size_t>(n_edges), 0,
                                            key_bits(n_nodes));
  return status == hipSuccess ? bytes : 0;
}

}  // namespace

size_t sort_workspace(int64_t n_edges, int64_t n_nodes) {
  if (n_edges <= 0 || n_nodes <= 0) return 0;
  const size_t pairs = rocprim_bytes(n_edges, n_nodes, true);
  const size_t keys = rocprim_bytes(n_edges, n_nodes, false);
  return round_up_256(static_cast<size_t>(n_edges) * sizeof(uint32_t)) + round_up_256(pairs > keys ? pairs : keys);
}

int sort_keys(const int64_t* keys, int64_t n_edges, int64_t n_nodes, uint32_t* sorted_keys, int64_t* order,
              void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (n_edges == 0) return DPA4K_OK;
  if (n_nodes > (int64_t(1) << 32)) return fail(DPA4K_EINVAL, "stable grouping supports at most 2^32 nodes");
  Carver carver{static_cast<char*>(workspace), workspace_bytes};
  uint32_t* keys_in = carver.take<uint32_t>(static_cast<size_t>(n_edges));
  size_t temp_bytes = rocprim_bytes(n_edges, n_nodes, order != nullptr);
  void* temp = carver.take<char>(temp_bytes);
  if (keys_in == nullptr || temp == nullptr) return fail(DPA4K_EWORKSPACE, "stable grouping: workspace too small");
  const int64_t blocks64 = (n_edges + 255) / 256;
  const unsigned int blocks = static_cast<unsigned int>(blocks64 > 8192 ? 8192 : blocks64);
  narrow_keys_kernel<<<blocks, 256, 0, stream>>>(keys, n_edges, keys_in);
  if (int s = launched("narrow_keys_kernel")) return s;
  if (order == nullptr)
    return hip_status(rocprim::radix_sort_keys(temp, temp_bytes, keys_in, sorted_keys, static_cast<size_t>(n_edges),
                                               0, key_bits(n_nodes), stream),
                      "rocprim::radix_sort_keys");
  rocprim::counting_iterator<int64_t> identity(0);
  return hip_status(rocprim::radix_sort_pairs(temp, temp_bytes, keys_in, sorted_keys, identity, order,
                                              static_cast<size_t>(n_edges), 0, key_bits(n_nodes), stream),
                    "rocprim::radix_sort_pairs");
}

}  // namespace dpa4k
