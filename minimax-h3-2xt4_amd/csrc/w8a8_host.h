// Host-side helpers of the C ABI: argument checks and the per-thread error
// message returned by w8a8_last_error().
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdarg.h>

#include <atomic>

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

// Compute units of device dev (0 <= dev < 64; cached per device).
inline int device_cus(int dev) {
  static std::atomic<int> cus[64];
  int n = cus[dev].load(std::memory_order_acquire);
  if (n > 0) return n;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
  cus[dev].store(n, std::memory_order_release);
  return n;
}

// Compute units of the current device (256 if it cannot be queried).
inline int current_device_cus() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  return device_cus(dev);
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
