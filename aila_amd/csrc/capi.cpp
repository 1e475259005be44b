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

int load_rope_pos(const aila_hip_rope_pos* rp, aila_hip_rope_pos* out, const char* what) {
  *out = aila_hip_rope_pos{};
  if (rp == nullptr) return AILA_HIP_OK;
  if (rp->prompt_pos_len < 0 && rp->prompt_pos_lens == nullptr)
    return set_error(AILA_HIP_EINVAL, "%s: prompt_pos_len=%d < 0", what, rp->prompt_pos_len);
  const bool mrope = rp->interleaved && rp->pos_t && rp->pos_h && rp->pos_w;
  if (mrope && (rp->pos_stride < 0 || rp->mrope_section_h < 0 || rp->mrope_section_w < 0))
    return set_error(AILA_HIP_EINVAL, "%s: bad mRoPE streams (pos_stride=%d sections h=%d w=%d)", what,
                     rp->pos_stride, rp->mrope_section_h, rp->mrope_section_w);
  *out = *rp;
  return AILA_HIP_OK;
}

}  // namespace aila

extern "C" const char* aila_hip_last_error(void) { return aila::g_last_error; }

extern "C" int aila_hip_version(void) { return (1 << 16) | 2; }
