// Library-wide entry points of the C ABI: version, error reporting and the
// status plumbing every kernel file uses.
#include <stdarg.h>
#include <stdio.h>

#include <atomic>

#include "api.h"

namespace {
thread_local char g_error[1024] = "";
}

namespace pk {

int fail(int status, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return status;
}

int cu_count() {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n > 0) return n;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
  cached[dev].store(n, std::memory_order_relaxed);
  return n;
}

int launched(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(PK_ERR_HIP, "%s: launch failed: %s", what, hipGetErrorString(err));
  g_error[0] = '\0';
  return PK_OK;
}

}  // namespace pk

extern "C" {

int pk_version(void) { return PK_ABI_VERSION; }

const char* pk_last_error(void) { return g_error; }

}  // extern "C"
