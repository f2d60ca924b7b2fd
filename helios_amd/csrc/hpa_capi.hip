// Error reporting and version entry points of the C-ABI.
#include <stdio.h>
#include <string.h>

#include "hpa_host.h"

namespace hpa {

static thread_local char g_err[512];

int fail(int status, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return status;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(HPA_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(e));
  return HPA_OK;
}

}  // namespace hpa

extern "C" const char* hpa_last_error(void) { return hpa::g_err; }

extern "C" int hpa_version(void) { return HPA_VERSION; }
