// Library identity and thread-local error reporting for the C ABI.
#include <stdarg.h>
#include <stdio.h>

#include "lc_common.h"

namespace {
thread_local char g_last_error[512] = "";
}

int lc_fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int lc_check_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    lc_fail(static_cast<int>(err), "%s: launch failed: %s", what, hipGetErrorString(err));
    return static_cast<int>(err);
  }
  return LC_OK;
}

int lc_cu_count() {
  static int cached = 0;
  if (cached == 0) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
      cached = n;
    else
      cached = 256;
  }
  return cached;
}

extern "C" {

// Major * 10000 + minor * 100 + patch.
int lc_version(void) { return 200; }

const char* lc_last_error(void) { return g_last_error; }

}  // extern "C"
