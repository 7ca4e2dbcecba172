#include "host_common.h"

#include <stdarg.h>
#include <stdio.h>

#include <atomic>
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

static std::atomic<unsigned long long> g_wait_ticks{10000000ull};  // 100 ms at 100 MHz

unsigned long long merge_wait_ticks() { return g_wait_ticks.load(std::memory_order_relaxed); }

int read_and_clear_ws_flags(void* workspace, hipStream_t stream, unsigned* flags) {
  hipError_t e = hipStreamSynchronize(stream);
  if (e != hipSuccess) return fail((int)e, "workspace_check: %s", hipGetErrorString(e));
  unsigned word = 0;
  e = hipMemcpyAsync(&word, workspace, sizeof(word), hipMemcpyDeviceToHost, stream);
  if (e == hipSuccess) e = hipStreamSynchronize(stream);
  if (e != hipSuccess) return fail((int)e, "workspace_check: read: %s", hipGetErrorString(e));
  if (flags) *flags = word;
  if (word == 0) return RLSE_OK;
  e = hipMemsetAsync(workspace, 0, sizeof(word), stream);
  if (e == hipSuccess) e = hipStreamSynchronize(stream);
  if (e != hipSuccess) return fail((int)e, "workspace_check: clear: %s", hipGetErrorString(e));
  if (word & RLSE_WS_ERR_MERGE_TIMEOUT)
    return fail(RLSE_ERR_DEVICE_TIMEOUT,
                "a merge on the device gave up waiting for a partial (flags 0x%x)", word);
  if (word & RLSE_WS_ERR_LENGTH)
    return fail(RLSE_ERR_TOKEN_LIMIT,
                "a sequence length exceeded its block table (flags 0x%x)", word);
  if (word & RLSE_WS_ERR_PREFIX)
    return fail(RLSE_ERR_INVALID_VALUE,
                "a cascade step's batch does not share its prefix pages, or a new token lies "
                "inside them (flags 0x%x)", word);
  return fail(RLSE_ERR_DEVICE_TIMEOUT, "unknown device error flags 0x%x", word);
}

}  // namespace rlse

extern "C" int rlse_set_merge_wait_ns(unsigned long long ns) {
  rlse::g_wait_ticks.store(ns / 10, std::memory_order_relaxed);  // 100 MHz: 10 ns per tick
  return RLSE_OK;
}

extern "C" const char* rlse_last_error(void) { return rlse::g_last_error; }

extern "C" int rlse_version(void) { return 200; /* 0.2.0 */ }
