// Error reporting shared by the C-ABI entry points.
#pragma once

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>

#include "../../include/drama3_moe.h"

namespace d3 {

int set_error(int code, const char* fmt, ...);
void clear_error();

inline hipStream_t as_stream(void* stream) { return reinterpret_cast<hipStream_t>(stream); }

}  // namespace d3

// Argument checks: return D3_ERR_INVALID_ARGUMENT with a message.
#define D3_REQUIRE(cond, ...)                                            \
  do {                                                                   \
    if (!(cond)) return ::d3::set_error(D3_ERR_INVALID_ARGUMENT, __VA_ARGS__); \
  } while (0)

#define D3_SUPPORTED(cond, ...)                                          \
  do {                                                                   \
    if (!(cond)) return ::d3::set_error(D3_ERR_UNSUPPORTED, __VA_ARGS__); \
  } while (0)

// After a kernel launch: surface launch-configuration errors.
#define D3_LAUNCHED(name)                                                           \
  do {                                                                              \
    hipError_t launch_status_ = hipGetLastError();                                  \
    if (launch_status_ != hipSuccess)                                               \
      return ::d3::set_error(D3_ERR_HIP, "%s launch failed: %s", name,              \
                             hipGetErrorString(launch_status_));                    \
    ::d3::clear_error();                                                            \
    return D3_OK;                                                                   \
  } while (0)
