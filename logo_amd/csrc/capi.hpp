// Host-side helpers shared by the C-ABI entry points: error recording and
// launch checking.
#pragma once

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>

#include "../../include/logo_hip.h"

namespace logo {

void set_error(const char* fmt, ...);

#define LOGO_REQUIRE(cond, ...)          \
  do {                                   \
    if (!(cond)) {                       \
      ::logo::set_error(__VA_ARGS__);    \
      return LOGO_EINVAL;                \
    }                                    \
  } while (0)

#define LOGO_HIP_CHECK(expr)                                                          \
  do {                                                                                \
    hipError_t err_ = (expr);                                                         \
    if (err_ != hipSuccess) {                                                         \
      ::logo::set_error("%s failed: %s", #expr, hipGetErrorString(err_));             \
      return LOGO_EHIP;                                                               \
    }                                                                                 \
  } while (0)

#define LOGO_LAUNCH_CHECK(name)                                                       \
  do {                                                                                \
    hipError_t err_ = hipGetLastError();                                              \
    if (err_ != hipSuccess) {                                                         \
      ::logo::set_error("launch of %s failed: %s", name, hipGetErrorString(err_));    \
      return LOGO_EHIP;                                                               \
    }                                                                                 \
  } while (0)

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

}  // namespace logo
