// Host-side helpers shared by the C-ABI entry points: status codes, the
// per-thread last-error message and HIP error checking.
#pragma once

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/nanochat_filter_amd.h"

namespace ltv {

void set_error(const char* fmt, ...);

#define LTV_REQUIRE(cond, code, ...)     \
  do {                                   \
    if (!(cond)) {                       \
      ::ltv::set_error(__VA_ARGS__);     \
      return (code);                     \
    }                                    \
  } while (0)

#define LTV_HIP_CHECK(expr)                                                         \
  do {                                                                              \
    hipError_t _e = (expr);                                                         \
    if (_e != hipSuccess) {                                                         \
      ::ltv::set_error("%s failed: %s (%s:%d)", #expr, hipGetErrorString(_e),       \
                       __FILE__, __LINE__);                                         \
      return LTV_ERR_HIP;                                                           \
    }                                                                               \
  } while (0)

// Launch-error check right after a kernel launch.
#define LTV_LAUNCH_CHECK() LTV_HIP_CHECK(hipGetLastError())

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline int next_pow2(int x) {
  int p = 1;
  while (p < x) p <<= 1;
  return p;
}

inline bool is_pow2(int x) { return x > 0 && (x & (x - 1)) == 0; }

}  // namespace ltv
