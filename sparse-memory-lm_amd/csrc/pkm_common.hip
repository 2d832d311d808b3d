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

// The device address of pinned host memory (hipHostMalloc, e.g. torch's pin_memory=True), so that a value table
// kept in host RAM is read by the same gather kernels over the host link (zero-copy).  Anything else -- pageable
// memory, device memory, unknown pointers -- is refused, so a kernel never gets an address the GPU cannot map.
extern "C" int smlm_host_table_pointer(const void *host, void **device) {
  using namespace smlm;
  if (!host || !device) return fail(SMLM_EINVAL, "smlm_host_table_pointer: null pointer argument");
  *device = nullptr;
  hipPointerAttribute_t attr;
  hipError_t e = hipPointerGetAttributes(&attr, host);
  if (e != hipSuccess) {
    (void)hipGetLastError();  // an unknown (pageable) pointer: clear the sticky error
    return fail(SMLM_EINVAL, "smlm_host_table_pointer: %p is not pinned host memory (%s)", host,
                hipGetErrorString(e));
  }
  if (attr.type != hipMemoryTypeHost || !attr.devicePointer)
    return fail(SMLM_EINVAL, "smlm_host_table_pointer: %p is not pinned host memory mapped for the device", host);
  *device = attr.devicePointer;
  return SMLM_OK;
}
