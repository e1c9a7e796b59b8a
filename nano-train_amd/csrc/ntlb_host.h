// Host-side helpers for the C-ABI launchers: thread-local error text and
// launch checking.  Every entry point validates its arguments before any
// launch and maps HIP runtime errors to NTLB_ELAUNCH.
#pragma once
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/ntlowbit.h"

namespace ntlb {

void set_error(const char* fmt, ...);
void clear_error();

inline int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  set_error("%s", buf);
  return code;
}

inline int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(NTLB_ELAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return NTLB_OK;
}

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

inline int dtype_size(int dt) { return dt == NTLB_F32 ? 4 : 2; }

inline bool valid_dtype(int dt) { return dt == NTLB_F32 || dt == NTLB_BF16 || dt == NTLB_F16; }

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// number of workgroups for grid-stride loops: enough to fill 256 CUs many
// times over without launching more groups than there is work
inline unsigned grid_for(int64_t work_items, int64_t items_per_group, int64_t max_groups = 256 * 16) {
  int64_t g = cdiv(work_items, items_per_group);
  if (g < 1) g = 1;
  if (g > max_groups) g = max_groups;
  return (unsigned)g;
}

}  // namespace ntlb
