// Host-side helpers of the C ABI: the thread-local error message, argument checks and launch checks.
#pragma once

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/sglang_neuron_amd.h"

namespace sna {

// The calling thread's last error message (defined in capi.hip).
char* error_buffer();
constexpr int kErrorBufferBytes = 512;

// Clears the thread's error message on entry of an API call.
struct ApiGuard {
  ApiGuard() { error_buffer()[0] = '\0'; }
};

__attribute__((format(printf, 2, 3))) inline int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(error_buffer(), kErrorBufferBytes, fmt, ap);
  va_end(ap);
  return code;
}

inline int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(SNA_ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return SNA_OK;
}

inline bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p % a) == 0; }

// Diagnostics timer (capi.hip): when sna_diag_kernel_timing(1) has switched it on, a decode launcher records an event
// before its split-K kernel (phase 0), between it and the combine pass (phase 1) and after the combine (phase 2).
void timing_mark(int phase, hipStream_t s);

}  // namespace sna
