// Status reporting and device queries shared by every C-ABI entry point.
#include <stdarg.h>
#include <stdio.h>

#include <functional>
#include <mutex>

#include "ss_common.h"

namespace {
thread_local char g_last_error[512] = "";
std::mutex g_cu_mutex;
int g_cu_count[64] = {0};

// Per device: one non-blocking side stream (default priority) and the two events
// of a fork/join, created on first use and kept for the life of the process.
struct SideStream {
  hipStream_t stream = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
};
std::mutex g_side_mutex;
SideStream g_side[64];
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

int run_concurrently(hipStream_t stream, const std::function<int(hipStream_t)>& side_work,
                     const std::function<int(hipStream_t)>& main_work) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    set_error("concurrent launch: no current HIP device");
    return SS_ERR_LAUNCH;
  }
  // The whole fork/join is enqueued under one lock: the events are shared, and a
  // wait enqueued on an event binds to the record that precedes it.
  std::lock_guard<std::mutex> lock(g_side_mutex);
  SideStream& ss = g_side[dev];
  if (!ss.stream) {
    if (hipStreamCreateWithFlags(&ss.stream, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreateWithFlags(&ss.fork, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&ss.join, hipEventDisableTiming) != hipSuccess) {
      set_error("concurrent launch: cannot create the side stream or its events");
      return SS_ERR_LAUNCH;
    }
  }
  if (hipEventRecord(ss.fork, stream) != hipSuccess || hipStreamWaitEvent(ss.stream, ss.fork, 0) != hipSuccess) {
    set_error("concurrent launch: fork failed");
    return SS_ERR_LAUNCH;
  }
  const int st_side = side_work(ss.stream);
  const bool recorded = hipEventRecord(ss.join, ss.stream) == hipSuccess;
  const int st_main = st_side == SS_OK ? main_work(stream) : st_side;
  // join after main_work is enqueued (and also when a launch failed), so work
  // enqueued on `stream` later never races the side stream
  const bool joined = recorded && hipStreamWaitEvent(stream, ss.join, 0) == hipSuccess;
  if (st_main != SS_OK) return st_main;
  if (!joined) {
    set_error("concurrent launch: join failed");
    return SS_ERR_LAUNCH;
  }
  return SS_OK;
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
