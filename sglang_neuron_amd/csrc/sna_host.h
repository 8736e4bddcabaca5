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
  if (plan->work_n < 0 || plan->work_n > SNA_MAX_WORK_MAP || plan->work_n > plan->n_work ||
      (plan->work_n > 0 && B > SNA_MAX_WORK_MAP))
    return fail(SNA_ERR_INVALID_ARGUMENT, "%s: plan item map of %d entries (n_work %d, B %d; at most %d)", what,
                plan->work_n, plan->n_work, B, SNA_MAX_WORK_MAP);
  // entries: row << 6 | split, the last split of a row flagged; a row's items consecutive, splits 0, 1, ... in order
  auto row_of = [](uint32_t e) { return (e & ~kWorkLastSplit) >> 6; };
  for (int32_t i = 0; i < plan->work_n; ++i) {
    const uint32_t e = plan->work[i];
    if ((int64_t)row_of(e) >= B || (int32_t)(e & 63u) >= (plan->max_splits > 1 ? plan->max_splits : 1))
      return fail(SNA_ERR_INVALID_ARGUMENT, "%s: plan item %d names row %u split %u (B %d, max_splits %d)", what, i,
                  row_of(e), e & 63u, B, plan->max_splits);
    const uint32_t prev = i > 0 ? plan->work[i - 1] : 0u;
    const bool next_split = i > 0 && row_of(prev) == row_of(e) && (prev & 63u) + 1 == (e & 63u);
    const bool new_row = (e & 63u) == 0 && (i == 0 || row_of(prev) < row_of(e));
    const bool last = i + 1 == plan->work_n || row_of(plan->work[i + 1]) != row_of(e);
    if ((!next_split && !new_row) || ((e & kWorkLastSplit) != 0) != last)
      return fail(SNA_ERR_INVALID_ARGUMENT, "%s: plan item %d (row %u split %u) is out of order or mis-flagged", what,
                  i, row_of(e), e & 63u);
  }
  return SNA_OK;
}

}  // namespace sna
