// Library-wide entry points: version and per-thread last error.
#include <stdio.h>

#include "host.hpp"

namespace {
thread_local char g_last_error[512] = "";
}

int gse_fail(int code, const char* msg) {
  snprintf(g_last_error, sizeof(g_last_error), "%s", msg);
  return code;
}

int gse_launch_check(const char* what) {
  hipError_t e = hipGetLastError();
  if (e == hipSuccess) return GSE_OK;
  snprintf(g_last_error, sizeof(g_last_error), "%s: launch failed: %s", what, hipGetErrorString(e));
  return GSE_ELAUNCH;
}

int gse_device_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cached[dev]) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    cached[dev] = cus;
  }
  return cached[dev];
}

extern "C" int gse_version(void) { return 100; }

extern "C" const char* gse_last_error(void) { return g_last_error; }
