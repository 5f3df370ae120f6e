// Error plumbing and device queries behind the C ABI (include/tileinfer_amd.h).
#include <stdarg.h>
#include <stdio.h>

#include <mutex>
#include <vector>

#include "ti_common.h"

namespace ti {

namespace {
thread_local char g_last_error[512] = "";
}

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    return fail(TI_ELAUNCH, "%s: launch failed: %s", what, hipGetErrorString(err));
  }
  return TI_OK;
}

int device_cu_count() {
  static std::mutex mu;
  static std::vector<int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  std::lock_guard<std::mutex> lock(mu);
  if (dev >= static_cast<int>(cache.size())) cache.resize(dev + 1, 0);
  if (cache[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0) {
      n = 256;  // MI355X
    }
    cache[dev] = n;
  }
  return cache[dev];
}

}  // namespace ti

extern "C" const char* ti_last_error(void) { return ti::g_last_error; }

extern "C" int32_t ti_abi_version(void) { return 7; }
