// Host-side runtime pieces of libpagedattn: error reporting, device queries.
#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <string>
#include <vector>

#include "common.h"

namespace pa {

namespace {
thread_local std::string g_last_error;
}

int set_error(int code, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    return set_error(PAGEDATTN_ERR_HIP, "%s: kernel launch failed: %s", what,
                     hipGetErrorString(e));
  }
  return PAGEDATTN_OK;
}

int device_cu_count() {
  static std::mutex mu;
  static std::vector<int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  std::lock_guard<std::mutex> lock(mu);
  if ((int)cache.size() <= dev) cache.resize(dev + 1, 0);
  if (cache[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount,
                              dev) != hipSuccess)
      return 0;
    cache[dev] = n;
  }
  return cache[dev];
}

}  // namespace pa

extern "C" {

int pagedattn_abi_version(void) { return PAGEDATTN_ABI_VERSION; }

const char* pagedattn_last_error(void) { return pa::g_last_error.c_str(); }

int pagedattn_device_cu_count(void) { return pa::device_cu_count(); }

}  // extern "C"
