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

}  // namespace dpa4k

extern "C" const char* dpa4k_last_error(void) { return dpa4k::g_message; }

extern "C" int dpa4k_abi_version(void) { return DPA4K_ABI_VERSION; }
