// Host-side helpers of the C ABI: argument checks and the per-thread error
// message returned by w8a8_last_error().
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdarg.h>

#include "w8a8.h"

namespace w8a8 {

void set_error(const char* fmt, ...);

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

inline int elem_size(int dt) {
  switch (dt) {
    case W8A8_F16: case W8A8_BF16: return 2;
    case W8A8_F32: case W8A8_I32: return 4;
    case W8A8_I8: return 1;
    default: return 0;
  }
}

inline int launch_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return W8A8_ERR_LAUNCH;
  }
  return W8A8_OK;
}

}  // namespace w8a8

#define W8A8_REQUIRE(cond, ...)              \
  do {                                       \
    if (!(cond)) {                           \
      ::w8a8::set_error(__VA_ARGS__);        \
      return W8A8_ERR_INVALID;               \
    }                                        \
  } while (0)
