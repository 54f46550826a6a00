// Library-wide state: per-thread error message, version, device queries.
#include <stdarg.h>
#include <stdio.h>

#include <mutex>
#include <vector>

#include "lz_common.h"

static thread_local char g_last_error[512] = "";

int lz_set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int lz_check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return lz_set_error(LZ_ELAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return LZ_OK;
}

int lz_num_cus() {
  static std::mutex mu;
  static std::vector<int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  std::lock_guard<std::mutex> lock(mu);
  if ((int)cache.size() <= dev) cache.resize(dev + 1, 0);
  if (cache[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev] = n;
  }
  return cache[dev];
}

LZ_EXPORT const char* lz_last_error(void) { return g_last_error; }

LZ_EXPORT int lz_version(void) { return 1; }

LZ_EXPORT int lz_device_cus(void) { return lz_num_cus(); }
