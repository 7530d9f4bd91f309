// Host-side helpers shared by the C-ABI entry points: error state, argument
// checks and launch checks.  Every entry point returns an sva_status (0 = ok)
// and leaves a message readable through sva_last_error().
#pragma once
#include <hip/hip_runtime.h>
#include <mutex>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/sva_hip.h"

namespace sva {
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();
int device_cu_count();
}  // namespace sva

#define SVA_REQUIRE(cond, ...)          \
  do {                                  \
    if (!(cond)) {                      \
      sva::set_error(__VA_ARGS__);      \
      return SVA_ERR_INVALID_ARGUMENT;  \
    }                                   \
  } while (0)

#define SVA_UNSUPPORTED(cond, ...)      \
  do {                                  \
    if (!(cond)) {                      \
      sva::set_error(__VA_ARGS__);      \
      return SVA_ERR_UNSUPPORTED;       \
    }                                   \
  } while (0)

#define SVA_CHECK_LAUNCH(name)                                                   \
  do {                                                                           \
    hipError_t e_ = hipGetLastError();                                           \
    if (e_ != hipSuccess) {                                                      \
      sva::set_error("%s launch failed: %s", name, hipGetErrorString(e_));       \
      return SVA_ERR_HIP;                                                        \
    }                                                                            \
  } while (0)

#define SVA_CHECK_HIP(expr, name)                                                \
  do {                                                                           \
    hipError_t e_ = (expr);                                                      \
    if (e_ != hipSuccess) {                                                      \
      sva::set_error("%s: %s", name, hipGetErrorString(e_));                     \
      return SVA_ERR_HIP;                                                        \
    }                                                                            \
  } while (0)

// Raises a kernel's dynamic LDS limit on its first launch.  The flag is a
// std::once_flag, so host threads launching at once set it exactly once; the
// call's result is kept and checked on every launch.
#define SVA_SET_MAX_LDS_ONCE(fn, bytes, name)                                                    \
  do {                                                                                           \
    static std::once_flag once_;                                                                 \
    static hipError_t err_ = hipSuccess;                                                         \
    std::call_once(once_, [] {                                                                   \
      err_ = hipFuncSetAttribute((const void*)(fn), hipFuncAttributeMaxDynamicSharedMemorySize, \
                                 (int)(bytes));                                                  \
    });                                                                                          \
    SVA_CHECK_HIP(err_, name);                                                                   \
  } while (0)
