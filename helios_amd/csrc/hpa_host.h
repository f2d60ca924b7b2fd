// Host-side helpers shared by the C-ABI translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>

#include "helios_attn.h"

namespace hpa {

// Records a printf-style message for hpa_last_error() and returns `status`.
int fail(int status, const char* fmt, ...);

// Turns a pending launch error into HPA_ERR_LAUNCH with a message.
int check_launch(const char* what);

inline int ilog2_exact(int x) {
  if (x <= 0 || (x & (x - 1))) return -1;
  int r = 0;
  while ((1 << r) < x) ++r;
  return r;
}

inline bool valid_dtype(int dt) { return dt >= HPA_F32 && dt <= HPA_I8; }

}  // namespace hpa
