// Row quantisation of the value table for the inference bag (int8 and packed 4-bit, one fp16 scale per row).
// The scheme is the one of scripts/quantize_table_eval.py:45-61 (int8) and smlm/kernels.py:280-300 (q4):
//   m    = the row's value of largest magnitude (the first one on ties, as torch.argmax)
//   d    = fp16(m / lo), replaced by 1 if it is zero
//   code = clamp(round_half_even(w / d), lo, hi)            (fp32 division, correctly rounded)
// int8: (lo, hi) = (-128, 127), codes stored as int8.  q4: (lo, hi) = (-8, 7), byte i of a row holds column i
// in the low nibble and column i + D/2 in the high nibble, each as code + 8.
// One wavefront per row; four rows per workgroup.
#include "pkm_common.h"

namespace smlm {
namespace {

template <bool SRC_F32>
__device__ __forceinline__ float src_val(const void *src, int64_t o) {
  if constexpr (SRC_F32) return ((const float *)src)[o];
  else return bf16_bits_to_f32(((const uint16_t *)src)[o]);
}

template <bool SRC_F32, bool Q4>
__global__ void __launch_bounds__(256) quantize_kernel(const void *__restrict__ src, int64_t rows, int D,
                                                       void *__restrict__ codes, uint16_t *__restrict__ scales) {
  const int64_t row = (int64_t)blockIdx.x * 4 + threadIdx.x / kWave;
  if (row >= rows) return;
  const int lane = lane_id();
  const int64_t base = row * D;

  float best = -1.f;
  int bi = 0x7FFFFFFF;
  for (int col = lane; col < D; col += kWave) {
    const float a = fabsf(src_val<SRC_F32>(src, base + col));
    if (a > best) { best = a; bi = col; }
  }
  for (int o = kWave / 2; o > 0; o >>= 1) {
    const float ob = __shfl_xor(best, o, kWave);
    const int oi = __shfl_xor(bi, o, kWave);
    if (ob > best || (ob == best && oi < bi)) { best = ob; bi = oi; }
  }
  if (bi >= D) bi = 0;  // a row without any ordered value (all NaN) still reads in bounds
  const float lo = Q4 ? -8.f : -128.f, hi = Q4 ? 7.f : 127.f;
  const float m = src_val<SRC_F32>(src, base + bi);
  uint16_t db = f32_to_f16_bits(m / lo);
  if ((db & 0x7FFFu) == 0) db = 0x3C00u;  // fp16 1.0
  const float d = f16_bits_to_f32(db);
  if (lane == 0) scales[row] = db;

  if constexpr (!Q4) {
    int8_t *out = (int8_t *)codes + base;
    for (int col = lane; col < D; col += kWave)
      out[col] = (int8_t)fminf(fmaxf(rintf(src_val<SRC_F32>(src, base + col) / d), lo), hi);
  } else {
    const int half = D / 2;
    uint8_t *out = (uint8_t *)codes + row * half;
    for (int col = lane; col < half; col += kWave) {
      const int c0 = (int)fminf(fmaxf(rintf(src_val<SRC_F32>(src, base + col) / d), lo), hi) + 8;
      const int c1 = (int)fminf(fmaxf(rintf(src_val<SRC_F32>(src, base + half + col) / d), lo), hi) + 8;
      out[col] = (uint8_t)(c0 | (c1 << 4));
    }
  }
}

}  // namespace
}  // namespace smlm

extern "C" int smlm_pkm_quantize(const void *src, int src_dtype, int64_t rows, int D, int kind, void *codes,
                                 uint16_t *scales, void *stream) {
  using namespace smlm;
  if (!src || !codes || !scales) return fail(SMLM_EINVAL, "smlm_pkm_quantize: null src, codes or scales pointer");
  if (src_dtype != SMLM_F32 && src_dtype != SMLM_BF16)
    return fail(SMLM_EINVAL, "smlm_pkm_quantize: src_dtype must be SMLM_F32 or SMLM_BF16, got %d", src_dtype);
  if (kind != SMLM_I8 && kind != SMLM_Q4)
    return fail(SMLM_EINVAL, "smlm_pkm_quantize: kind must be SMLM_I8 or SMLM_Q4, got %d", kind);
  if (rows < 0 || D < 1 || (kind == SMLM_Q4 && D % 2))
    return fail(SMLM_EINVAL, "smlm_pkm_quantize: bad shape rows=%lld D=%d", (long long)rows, D);
  if (rows == 0) return SMLM_OK;
  const int64_t blocks = (rows + 3) / 4;
  if (blocks > 0x7FFFFFFFLL) return fail(SMLM_EINVAL, "smlm_pkm_quantize: rows=%lld too large", (long long)rows);
  const dim3 grid((unsigned)blocks), block(4 * kWave);
  hipStream_t s = (hipStream_t)stream;
  const bool f32 = src_dtype == SMLM_F32, q4 = kind == SMLM_Q4;
  if (f32 && q4) hipLaunchKernelGGL((quantize_kernel<true, true>), grid, block, 0, s, src, rows, D, codes, scales);
  else if (f32) hipLaunchKernelGGL((quantize_kernel<true, false>), grid, block, 0, s, src, rows, D, codes, scales);
  else if (q4) hipLaunchKernelGGL((quantize_kernel<false, true>), grid, block, 0, s, src, rows, D, codes, scales);
  else hipLaunchKernelGGL((quantize_kernel<false, false>), grid, block, 0, s, src, rows, D, codes, scales);
  return launch_status("smlm_pkm_quantize");
}
