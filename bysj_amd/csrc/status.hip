// Error plumbing of the C ABI: status codes plus a thread-local message.
#include <atomic>
#include <cstdarg>
#include <cstdio>

#include "common.h"

namespace dpa4k {
namespace {
thread_local char g_message[512] = "";
}  // namespace

void clear_error() { g_message[0] = '\0'; }

int fail(int code, const char* format, ...) {
  va_list args;
  va_start(args, format);
  std::vsnprintf(g_message, sizeof(g_message), format, args);
  va_end(args);
  return code;
}

int hip_status(hipError_t status, const char* what) {
  if (status == hipSuccess) return DPA4K_OK;
  return fail(DPA4K_EHIP, "%s failed: %s", what, hipGetErrorString(status));
}

int launched(const char* kernel) {
  const hipError_t status = hipGetLastError();
  if (status == hipSuccess) return DPA4K_OK;
  return fail(DPA4K_EHIP, "launch of %s failed: %s", kernel, hipGetErrorString(status));
}

namespace {
__global__ __launch_bounds__(256) void zero_fill_kernel(uint32_t* __restrict__ words, int64_t count) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < count; i += stride)
    words[i] = 0u;
}
}  // namespace

int zero_fill(void* pointer, size_t bytes, hipStream_t stream) {
  if (bytes == 0) return DPA4K_OK;
  if (pointer == nullptr || (bytes & 3u) != 0 || (reinterpret_cast<uintptr_t>(pointer) & 3u) != 0)
    return fail(DPA4K_EINVAL, "zero fill: null, unaligned or ragged buffer");
  const int64_t words = static_cast<int64_t>(bytes / 4);
  const int64_t blocks = (words + 255) / 256;
  const unsigned int grid = static_cast<unsigned int>(blocks < 4096 ? blocks : 4096);
  zero_fill_kernel<<<grid, 256, 0, stream>>>(static_cast<uint32_t*>(pointer), words);
  return launched("zero_fill_kernel");
}

namespace {
// 0: the hardware limit.  Only dpa4k_set_launch_row_limit changes it.
std::atomic<int64_t> g_row_limit{0};
}  // namespace

int64_t row_block_limit(int threads) {
  const int64_t hardware = 4294967295LL / threads;
  const int64_t lowered = g_row_limit.load(std::memory_order_relaxed);
  return lowered > 0 && lowered < hardware ? lowered : hardware;
}

}  // namespace dpa4k

extern "C" int dpa4k_set_launch_row_limit(int64_t blocks) {
  dpa4k::clear_error();
  if (blocks < 0) return dpa4k::fail(DPA4K_EINVAL, "launch row limit must be non-negative");
  dpa4k::g_row_limit.store(blocks, std::memory_order_relaxed);
  return DPA4K_OK;
}

extern "C" const char* dpa4k_last_error(void) { return dpa4k::g_message; }

extern "C" int dpa4k_abi_version(void) { return DPA4K_ABI_VERSION; }
