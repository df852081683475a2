// Status codes and the thread-local error message behind wq_last_error().
#pragma once

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>

#include "ondeviceinfer_wq.h"

namespace wq {

void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));

inline int fail(int status, const char* what) {
  set_error("%s", what);
  return status;
}

// Every launch is followed by hipGetLastError so an invalid configuration is
// reported by the call that caused it.
inline int check_launch(const char* kernel) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s launch failed: %s", kernel, hipGetErrorString(e));
    return WQ_ERR_HIP;
  }
  return WQ_OK;
}

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

}  // namespace wq

#define WQ_REQUIRE(cond, status, ...)            \
  do {                                           \
    if (!(cond)) {                               \
      ::wq::set_error(__VA_ARGS__);              \
      return (status);                           \
    }                                            \
  } while (0)
