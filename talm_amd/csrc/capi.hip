// Status reporting of the C-ABI (talm_last_error, talm_abi_version) and device queries.
#include <atomic>
#include <cstdarg>
#include <cstdio>

#include "common.h"

namespace {
thread_local char g_error[512] = "";
}

namespace talm {

int fail(int status, const char* fmt, ...) {
  va_list args;
  va_start(args, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, args);
  va_end(args);
  return status;
}

int ok() {
  g_error[0] = '\0';
  return TALM_OK;
}

int check_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(TALM_EHIP, "%s: %s", what, hipGetErrorString(err));
  return ok();
}

int device_cus() {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n > 0) return n;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 1)
    n = 256;
  cached[dev].store(n, std::memory_order_relaxed);
  return n;
}

}  // namespace talm

TALM_API const char* talm_last_error(void) { return g_error; }

TALM_API int talm_abi_version(void) { return 20; }
