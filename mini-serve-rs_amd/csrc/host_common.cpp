#include "host_common.h"

#include <stdarg.h>
#include <stdio.h>

#include <mutex>
#include <vector>

namespace rlse {

static thread_local char g_last_error[512] = {0};

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_last_error[0] = 0; }

size_t dtype_size(int dtype) {
  switch (dtype) {
    case RLSE_DTYPE_F32:
      return 4;
    case RLSE_DTYPE_BF16:
    case RLSE_DTYPE_F16:
      return 2;
    default:
      return 0;
  }
}

int launch_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail((int)e, "%s: launch failed: %s", what, hipGetErrorString(e));
  return RLSE_OK;
}

int device_cu_count(int* cus) {
  static std::mutex mu;
  static std::vector<int> cache;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail((int)e, "hipGetDevice: %s", hipGetErrorString(e));
  std::lock_guard<std::mutex> lock(mu);
  if ((int)cache.size() <= dev) cache.resize(dev + 1, 0);
  if (cache[dev] == 0) {
    int n = 0;
    e = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return fail((int)e, "hipDeviceGetAttribute: %s", hipGetErrorString(e));
    cache[dev] = n;
  }
  *cus = cache[dev];
  return RLSE_OK;
}

}  // namespace rlse

extern "C" const char* rlse_last_error(void) { return rlse::g_last_error; }

extern "C" int rlse_version(void) { return 100; /* 0.1.0 */ }
