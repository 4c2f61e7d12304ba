// Library-wide state of the kmoe C ABI: the thread-local error message and the
// launch-status check every entry point ends with.
#include <stdarg.h>

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

}  // namespace kmoe

extern "C" const char* kmoe_last_error(void) { return g_last_error; }

extern "C" int kmoe_abi_version(void) { return KMOE_ABI_VERSION; }
