// Error plumbing of the C ABI: status codes plus a thread-local message.
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

}  // namespace dpa4k

extern "C" const char* dpa4k_last_error(void) { return dpa4k::g_message; }

extern "C" int dpa4k_abi_version(void) { return DPA4K_ABI_VERSION; }
