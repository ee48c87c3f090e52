// Error reporting shared by the C-ABI entry points: every entry returns 0 on
// success or -1 after recording a message that fp_last_error() returns (per
// host thread).  Mirrors the reference's TORCH_CHECK / launch-check points.
#pragma once

#include <hip/hip_runtime.h>
#include <stdio.h>

namespace fp {
void set_error(const char* msg);
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
