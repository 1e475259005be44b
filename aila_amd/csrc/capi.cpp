// C-ABI plumbing: thread-local last-error message and version.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>

#include "aila_hip.h"

namespace aila {

static thread_local char g_last_error[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return set_error(AILA_HIP_ELAUNCH, "%s: %s", what, hipGetErrorString(e));
  g_last_error[0] = '\0';
  return AILA_HIP_OK;
}

}  // namespace aila

extern "C" const char* aila_hip_last_error(void) { return aila::g_last_error; }

extern "C" int aila_hip_version(void) { return (1 << 16) | 0; }
