// Status reporting shared by every extern "C" entry point: a failing call
// returns a negative OV_* code and leaves its message for ovh_last_error() on
// the calling thread; no exception crosses the C boundary.
#pragma once

#include <hip/hip_runtime.h>

#include <string>

namespace ovh {

int set_error(int code, const std::string& msg);  // returns code
int hip_error(hipError_t e, const char* what);    // OV_ERR_INTERNAL with hipGetErrorString

}  // namespace ovh

#define OVH_HIP(expr, what)                                   \
  do {                                                        \
    const hipError_t e_ = (expr);                             \
    if (e_ != hipSuccess) return ::ovh::hip_error(e_, what);  \
  } while (0)
