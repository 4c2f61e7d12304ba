// Library-wide state of the kmoe C ABI: the thread-local error message, the
// launch-status check every entry point ends with, and the per-device CU count
// that sizes persistent grids.
#include <stdarg.h>

#include <atomic>

#include "kmoe_common.h"

namespace {
thread_local char g_last_error[512] = "";
}

namespace kmoe {

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: HIP launch failed: %s", what, hipGetErrorString(e));
    return KMOE_ERR_LAUNCH;
  }
  return KMOE_OK;
}

int cu_count() {
  constexpr int kMaxDevices = 64;
  static std::atomic<int> cached[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 256;
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n > 0) return n;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
  cached[dev].store(n, std::memory_order_relaxed);
  return n;
}

}  // namespace kmoe

extern "C" const char* kmoe_last_error(void) { return g_last_error; }

extern "C" int kmoe_abi_version(void) { return KMOE_ABI_VERSION; }

extern "C" int kmoe_pack_layout_version(void) { return KMOE_PACK_LAYOUT; }
