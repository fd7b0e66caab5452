// Thread-local error reporting for the C ABI (atlas_last_error).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>

#include "atlas_scan.h"

namespace atlas {

char* error_buffer();  // thread-local, defined in atlas_abi.hip

inline void clear_error() { error_buffer()[0] = '\0'; }

__attribute__((format(printf, 2, 3))) inline atlas_status fail(atlas_status s, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(error_buffer(), 512, fmt, ap);
  va_end(ap);
  return s;
}

inline atlas_status fail_hip(hipError_t e, const char* what) {
  return fail(ATLAS_ERR_HIP, "%s: %s (%d)", what, hipGetErrorString(e), (int)e);
}

}  // namespace atlas
