// Error state and library-level entry points of the C ABI.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

#include <atomic>

namespace ssd {

static thread_local char g_err[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

static std::atomic<uint64_t> g_launches{0};
void count_launch() { g_launches.fetch_add(1, std::memory_order_relaxed); }

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(SSD_EHIP, "%s: launch failed: %s", what, hipGetErrorString(e));
  return SSD_OK;
}

}  // namespace ssd

SSD_API const char* ssd_last_error(void) { return ssd::g_err; }

SSD_API int ssd_abi_version(void) { return 6; }

// Kernels enqueued by this library since it was loaded (all devices and streams).
SSD_API uint64_t ssd_launch_count(void) { return ssd::g_launches.load(std::memory_order_relaxed); }

#ifndef SSD_BUILD_HASH
#define SSD_BUILD_HASH "unknown"
#endif
// Hash of the sources this library was built from (set by the build script); the Python loader
// compares it with the sources beside it and refuses a stale build.
SSD_API const char* ssd_build_hash(void) { return SSD_BUILD_HASH; }

SSD_API int ssd_device_arch(char* buf, int len) {
  int dev = 0;
  hipDeviceProp_t p;
  if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&p, dev) != hipSuccess)
    return ssd::set_error(ssd::SSD_EHIP, "no HIP device");
  snprintf(buf, len, "%s", p.gcnArchName);
  return ssd::SSD_OK;
}
