// The decode lookup (sub-key scores, then selection fused with the value bag) for callers that cannot allocate:
// the sub-key score rows s1, s2 -- the workspace that smlm_pkm_score writes and smlm_pkm_select_bag reads --
// live in a static device array of this file instead of caller-provided buffers.
#include <mutex>

#include "pkm_common.h"

namespace {

// One array per GPU the library runs on, alive until the process ends.  Host code never passes `scratch` itself
// to a kernel (its host-side name is not a device address): it uses the address hipGetSymbolAddress returns on
// each device.
__device__ __align__(256) unsigned char scratch[SMLM_LOOKUP_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void *g_scratch_ptr[kMaxDevices] = {};

// The device address of `scratch` on the current device, looked up on the first call on that device.
int scratch_pointer(void *stream, void **ptr) {
  using namespace smlm;
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess)
    return fail(SMLM_EHIP, "smlm_pkm_lookup_noalloc: hipGetDevice failed: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return fail(SMLM_EUNSUPPORTED, "smlm_pkm_lookup_noalloc: device %d is beyond the %d this library tracks", dev,
                kMaxDevices);
  if (stream) {
    int sdev = -1;
    e = hipStreamGetDevice((hipStream_t)stream, &sdev);
    if (e != hipSuccess)
      return fail(SMLM_EHIP, "smlm_pkm_lookup_noalloc: hipStreamGetDevice failed: %s", hipGetErrorString(e));
    if (sdev != dev)
      return fail(SMLM_EINVAL, "smlm_pkm_lookup_noalloc: the stream belongs to device %d, the current device is %d",
                  sdev, dev);
  }
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(SMLM_EHIP, "smlm_pkm_lookup_noalloc: hipGetSymbolAddress of the scratch array failed on device "
                  "%d: %s", dev, hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return SMLM_OK;
}

}  // namespace

extern "C" int smlm_pkm_lookup_noalloc(const void *q, int64_t q_row_stride, const void *keys, int dtype, int64_t N,
                                       int H, int NK, int half, int knn, const void *table, int table_dtype,
                                       int64_t rows, int D, const uint16_t *scales, const uint16_t *pre, void *out,
                                       int out_dtype, void *stream) {
  using namespace smlm;
  if (dtype != SMLM_BF16 && dtype != SMLM_F32)
    return fail(SMLM_EINVAL, "smlm_pkm_lookup_noalloc: dtype must be SMLM_BF16 or SMLM_F32, got %d", dtype);
  if (N < 0 || H < 1 || NK < 1)
    return fail(SMLM_EINVAL, "smlm_pkm_lookup_noalloc: bad shape N=%lld H=%d NK=%d", (long long)N, H, NK);
  if (N > (int64_t)SMLM_LOOKUP_SCRATCH_BYTES)
    return fail(SMLM_EUNSUPPORTED, "smlm_pkm_lookup_noalloc: N=%lld tokens exceed what the %lld-byte scratch "
                "array can hold", (long long)N, (long long)SMLM_LOOKUP_SCRATCH_BYTES);
  // every argument check of both steps before anything is sized or launched: with N = 0 they validate and return
  // (among them H <= 32768 and NK <= 65536, which keep the size below within int64)
  const void *fake = table ? table : q;
  int rc = smlm_pkm_score(q, q_row_stride, keys, dtype, 0, H, NK, half, (void *)fake, (void *)fake, stream);
  if (rc != SMLM_OK) return rc;
  rc = smlm_pkm_select_bag(fake, fake, dtype, 0, H, NK, knn, table, table_dtype, rows, D, scales, pre, out,
                           out_dtype, nullptr, nullptr, nullptr, stream);
  if (rc != SMLM_OK) return rc;
  // s1 at the start of the array, s2 at the next 256-byte boundary after it
  const int64_t elem = dtype == SMLM_F32 ? 4 : 2;
  const int64_t one = N * H * NK * elem;
  const int64_t s2_off = (one + 255) / 256 * 256;
  if (s2_off + one > (int64_t)SMLM_LOOKUP_SCRATCH_BYTES)
    return fail(SMLM_EUNSUPPORTED, "smlm_pkm_lookup_noalloc: N=%lld x H=%d x NK=%d scores need %lld bytes of "
                "scratch; the static array holds %lld (use smlm_pkm_score + smlm_pkm_select_bag with buffers of "
                "your own)", (long long)N, H, NK, (long long)(s2_off + one), (long long)SMLM_LOOKUP_SCRATCH_BYTES);
  if (N == 0) return SMLM_OK;
  void *base = nullptr;
  rc = scratch_pointer(stream, &base);
  if (rc != SMLM_OK) return rc;
  void *s1 = base, *s2 = (unsigned char *)base + s2_off;
  rc = smlm_pkm_score(q, q_row_stride, keys, dtype, N, H, NK, half, s1, s2, stream);
  if (rc != SMLM_OK) return rc;
  return smlm_pkm_select_bag(s1, s2, dtype, N, H, NK, knn, table, table_dtype, rows, D, scales, pre, out, out_dtype,
                             nullptr, nullptr, nullptr, stream);
}
