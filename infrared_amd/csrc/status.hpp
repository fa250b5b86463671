// Host-side status plumbing shared by the C-ABI entry points: a thread-local
// last-error message and argument checks that turn into IR_E* return codes.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "infrared_amd.h"

namespace ir {

// Records a printf-style message as this thread's last error; returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Clears the last error; returns IR_OK.
int ok();

// Maps the result of the preceding launches to IR_OK / IR_ELAUNCH.
int check_launch(const char* what);

// CUs of the current device, cached per device (256 if the runtime cannot say).
int device_cus();

// Accelerator complex dies (XCDs) of the current device, cached per device (1
// if the runtime cannot say). The dispatcher hands workgroup i of a launch to
// XCD i mod this count; each XCD has its own L2.
int device_xcds();

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

inline int dtype_bytes(int dtype) {
  switch (dtype) {
    case IR_DTYPE_F32: return 4;
    case IR_DTYPE_F16: return 2;
    case IR_DTYPE_BF16: return 2;
    default: return 0;
  }
}

}  // namespace ir

#define IR_REQUIRE(cond, ...)                                   \
  do {                                                          \
    if (!(cond)) return ::ir::fail(IR_EINVAL, __VA_ARGS__);     \
  } while (0)
