// Error state and library-level queries of the C ABI (include/bmx.h).
#include <stdarg.h>
#include <stdio.h>

#include "bmx_common.h"

namespace {
thread_local char g_last_error[512] = "";
}

namespace bmx {

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(BMX_ELAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  g_last_error[0] = '\0';
  return BMX_OK;
}

int device_cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    cached[dev] = cus;
  }
  return cached[dev];
}

}  // namespace bmx

extern "C" {

const char* bmx_last_error(void) { return g_last_error; }

int bmx_abi_version(void) { return 2; }

}  // extern "C"
