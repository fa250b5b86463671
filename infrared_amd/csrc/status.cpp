// Thread-local error state behind ir_last_error().
#include "status.hpp"

#include <stdarg.h>
#include <stdio.h>

#include <atomic>

namespace {
thread_local char g_last_error[512] = "";
}

namespace ir {

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int ok() {
  g_last_error[0] = '\0';
  return IR_OK;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(IR_ELAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return ok();
}

int device_cus() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

int device_xcds() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 1;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeNumberOfXccs, dev) != hipSuccess || n <= 0) n = 1;
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

}  // namespace ir

extern "C" const char* ir_last_error(void) { return g_last_error; }

extern "C" const char* ir_version(void) { return "infrared_amd 0.1 gfx950"; }

extern "C" int ir_stream_capture_id(ir_stream_t stream, uint64_t* capture_id) {
  IR_REQUIRE(capture_id, "ir_stream_capture_id: null pointer");
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  unsigned long long id = 0;
  const hipError_t e = hipStreamGetCaptureInfo((hipStream_t)stream, &st, &id);
  if (e != hipSuccess) return ir::fail(IR_ELAUNCH, "ir_stream_capture_id: %s", hipGetErrorString(e));
  *capture_id = st == hipStreamCaptureStatusActive ? (uint64_t)id + 1 : 0;
  return ir::ok();
}
