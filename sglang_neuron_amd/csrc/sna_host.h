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

// A plan's item map, checked before a kernel reads it from its arguments: at most SNA_MAX_WORK_MAP entries, no more
// than the plan's items, every row below B and every split below the plan's count (a kernel indexes seq_lens, the
// block table and the workspace with them).
inline int check_work_map(const sna_split_plan* plan, int32_t B, const char* what) {
  if (plan->work_n < 0 || plan->work_n > SNA_MAX_WORK_MAP || plan->work_n > plan->n_work)
    return fail(SNA_ERR_INVALID_ARGUMENT, "%s: plan item map of %d entries (n_work %d, at most %d)", what,
                plan->work_n, plan->n_work, SNA_MAX_WORK_MAP);
  for (int32_t i = 0; i < plan->work_n; ++i) {
    const uint32_t e = plan->work[i];
    if ((int64_t)(e >> 6) >= B || (int32_t)(e & 63u) >= (plan->max_splits > 1 ? plan->max_splits : 1))
      return fail(SNA_ERR_INVALID_ARGUMENT, "%s: plan item %d names row %u split %u (B %d, max_splits %d)", what, i,
                  e >> 6, e & 63u, B, plan->max_splits);
  }
  return SNA_OK;
}

}  // namespace sna
