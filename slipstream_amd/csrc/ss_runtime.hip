// Status reporting and device queries shared by every C-ABI entry point.
#include <stdarg.h>
#include <stdio.h>

#include <mutex>

#include "ss_common.h"

namespace {
thread_local char g_last_error[512] = "";
std::mutex g_cu_mutex;
int g_cu_count[64] = {0};
}  // namespace

namespace ss_host {

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

int launch_status(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    set_error("%s: HIP launch failed: %s", what, hipGetErrorString(err));
    return SS_ERR_LAUNCH;
  }
  return SS_OK;
}

int device_cu_count() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  std::lock_guard<std::mutex> lock(g_cu_mutex);
  if (g_cu_count[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    g_cu_count[dev] = n;
  }
  return g_cu_count[dev];
}

}  // namespace ss_host

extern "C" {

const char* ss_status_string(int status) {
  switch (status) {
    case SS_OK:
      return "ok";
    case SS_ERR_INVALID:
      return "invalid argument";
    case SS_ERR_UNSUPPORTED:
      return "unsupported shape or dtype";
    case SS_ERR_LAUNCH:
      return "HIP launch error";
    case SS_ERR_WORKSPACE:
      return "workspace too small";
    default:
      return "unknown status";
  }
}

const char* ss_last_error(void) { return g_last_error; }

int ss_version(void) { return 100; }

}  // extern "C"
