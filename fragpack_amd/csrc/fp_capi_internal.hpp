// Error reporting shared by the C-ABI entry points: every entry returns 0 on
// success or -1 after recording a message that fp_last_error() returns (per
// host thread).  Mirrors the reference's TORCH_CHECK / launch-check points.
#pragma once

#include <hip/hip_runtime.h>
#include <stdio.h>

namespace fp {
void set_error(const char* msg);

// Compute units of the current device (cached per device; 0 if unknown).
inline int device_cus() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (cache[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    cache[dev] = cus;
  }
  return cache[dev];
}
}  // namespace fp

#define FP_CHECK(cond, msg)   \
  do {                        \
    if (!(cond)) {            \
      ::fp::set_error(msg);   \
      return -1;              \
    }                         \
  } while (0)

#define FP_LAUNCH_CHECK()                                   \
  do {                                                      \
    hipError_t e_ = hipGetLastError();                      \
    if (e_ != hipSuccess) {                                 \
      ::fp::set_error(hipGetErrorString(e_));               \
      return -1;                                            \
    }                                                       \
  } while (0)
