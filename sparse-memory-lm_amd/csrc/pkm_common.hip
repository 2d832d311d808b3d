// Error state and version of the C ABI (include/smlm_pkm.h).
#include <stdarg.h>
#include <stdio.h>

#include "pkm_common.h"

namespace smlm {

static thread_local char g_last_error[512] = "";

int fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof g_last_error, fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_last_error[0] = '\0'; }

int launch_status(const char *what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(SMLM_EHIP, "%s: launch failed: %s", what, hipGetErrorString(e));
  return SMLM_OK;
}

}  // namespace smlm

extern "C" const char *smlm_pkm_version(void) { return "smlm_pkm 0.1.0 gfx950"; }

extern "C" const char *smlm_pkm_last_error(void) { return smlm::g_last_error; }
