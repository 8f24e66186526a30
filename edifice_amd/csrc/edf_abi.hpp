// Host-side helpers shared by the C-ABI entry points: status codes, the
// thread-local error string and launch checking.
#pragma once

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>

#include "../../include/edifice_hip.h"

namespace edf {

int set_error(int code, const char* fmt, ...);
int clear_error();

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Check the launch that was just issued; returns EDF_OK or EDF_ERR_LAUNCH.
inline int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(EDF_ERR_LAUNCH, "%s kernel launch failed: %s", what, hipGetErrorString(e));
  return clear_error();
}

inline bool valid_dtype(int dt) { return dt == EDF_F32 || dt == EDF_BF16; }

}  // namespace edf

#define EDF_REQUIRE(cond, code, ...)                         \
  do {                                                       \
    if (!(cond)) return ::edf::set_error((code), __VA_ARGS__); \
  } while (0)
