// Sub-key scoring (kernel 1) on the matrix cores: for every head h and half p,
//   s_p[n, h, k] = sum_{d < half} q[n, h, p*half + d] * keys[h, p, k, d]
// which is ProductKeyMemory.subkey_scores (smlm/pkm.py:117-123), a batched NT GEMM with M = sub-keys,
// N = tokens, K = half.  bf16 uses v_mfma_f32_16x16x32_bf16 (fp32 accumulation, bf16 result rounded to
// nearest even); fp32 uses v_mfma_f32_16x16x4_f32.
//
// Operand mapping (16x16 MFMA, 64 lanes, r = lane % 16, g = lane / 16):
//   A (sub-keys, 16 x Kstep):   lane holds key row r, the g-th 16-byte group of the step's dims
//   B (tokens, Kstep x 16):     lane holds token r, the same dims
//   D (16 x 16 fp32):           lane holds keys 4g..4g+3 of token r
// so every operand fetch is one 16-byte load per lane, and every lane stores 4 consecutive scores of one
// token.  For fp32 the 4 floats of a lane's 16 bytes feed 4 consecutive MFMAs: the contraction is a sum, so
// the order in which dims meet the hardware's k slots does not matter as long as A and B agree.
#include "pkm_common.h"

namespace smlm {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

template <bool F32, int WM, int WN, int WAVES_M, int WAVES_N>
__global__ void __launch_bounds__(WAVES_M *WAVES_N * 64)
    score_kernel(const void *__restrict__ q, int64_t q_stride, const void *__restrict__ keys, int N, int H, int NK,
                 int half, void *__restrict__ s1, void *__restrict__ s2) {
  constexpr int ESZ = F32 ? 4 : 2;
  constexpr int EPL = 16 / ESZ;      // elements per 16-byte load
  constexpr int KSTEP = 4 * EPL;     // dims consumed per step by the four lane groups
  const int z = blockIdx.z;
  const int h = z >> 1, p = z & 1;
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int wm = wave % WAVES_M, wn = wave / WAVES_M;
  const int key0 = blockIdx.y * (WAVES_M * WM * 16) + wm * WM * 16;
  const int tok0 = blockIdx.x * (WAVES_N * WN * 16) + wn * WN * 16;
  const int r = lane & 15, g = lane >> 4;

  const char *kbase = (const char *)keys + (int64_t)(h * 2 + p) * NK * half * ESZ;
  const char *qbase = (const char *)q + ((int64_t)h * 2 * half + (int64_t)p * half) * ESZ;

  floatx4 acc[WM][WN];
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int j = 0; j < WN; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  const uint4 zero = {0u, 0u, 0u, 0u};
  for (int k0 = 0; k0 < half; k0 += KSTEP) {
    const int kk = k0 + g * EPL;
    const bool kin = kk < half;  // half % EPL == 0: a lane's group is entirely inside or outside
    uint4 a[WM], b[WN];
#pragma unroll
    for (int i = 0; i < WM; ++i) {
      const int key = key0 + i * 16 + r;
      a[i] = (kin && key < NK) ? *(const uint4 *)(kbase + ((int64_t)key * half + kk) * ESZ) : zero;
    }
#pragma unroll
    for (int j = 0; j < WN; ++j) {
      const int tok = tok0 + j * 16 + r;
      b[j] = (kin && tok < N) ? *(const uint4 *)(qbase + ((int64_t)tok * q_stride + kk) * ESZ) : zero;
    }
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
      for (int j = 0; j < WN; ++j) {
        if constexpr (F32) {
          const float *fa = (const float *)&a[i];
          const float *fb = (const float *)&b[j];
#pragma unroll
          for (int s = 0; s < 4; ++s)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[s], fb[s], acc[i][j], 0, 0, 0);
        } else {
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a[i]),
                                                              __builtin_bit_cast(bf16x8, b[j]), acc[i][j], 0, 0, 0);
        }
      }
  }

  char *out = (char *)(p ? s2 : s1);
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int j = 0; j < WN; ++j) {
      const int tok = tok0 + j * 16 + r;
      const int key = key0 + i * 16 + g * 4;
      if (tok >= N || key >= NK) continue;
      const int64_t o = ((int64_t)tok * H + h) * NK + key;
      const floatx4 v = acc[i][j];
      if ((NK & 3) == 0 && key + 3 < NK) {  // 4 aligned consecutive scores
        if constexpr (F32) {
          *(floatx4 *)(out + o * 4) = v;
        } else {
          uint2 pk;
          pk.x = bf16_bits_rtne(v[0]) | (bf16_bits_rtne(v[1]) << 16);
          pk.y = bf16_bits_rtne(v[2]) | (bf16_bits_rtne(v[3]) << 16);
          *(uint2 *)(out + o * 2) = pk;
        }
      } else {
        for (int e = 0; e < 4 && key + e < NK; ++e) {
          if constexpr (F32) ((float *)out)[o + e] = v[e];
          else ((uint16_t *)out)[o + e] = (uint16_t)bf16_bits_rtne(v[e]);
        }
      }
    }
}

template <bool F32, int WM, int WN, int WAVES_M, int WAVES_N>
void launch_score(const void *q, int64_t q_stride, const void *keys, int64_t N, int H, int NK, int half, void *s1,
                  void *s2, hipStream_t stream) {
  constexpr int BM = WAVES_M * WM * 16, BN = WAVES_N * WN * 16;
  const dim3 grid((unsigned)((N + BN - 1) / BN), (unsigned)((NK + BM - 1) / BM), (unsigned)(2 * H));
  hipLaunchKernelGGL((score_kernel<F32, WM, WN, WAVES_M, WAVES_N>), grid, dim3(WAVES_M * WAVES_N * 64), 0, stream,
                     q, q_stride, keys, (int)N, H, NK, half, s1, s2);
}

template <bool F32>
void dispatch_score(const void *q, int64_t q_stride, const void *keys, int64_t N, int H, int NK, int half, void *s1,
                    void *s2, hipStream_t stream) {
  if (N <= 16)  // decode: 128 sub-keys x 16 tokens per workgroup, spread over many workgroups
    launch_score<F32, 2, 1, 4, 1>(q, q_stride, keys, N, H, NK, half, s1, s2, stream);
  else          // 128 sub-keys x 64 tokens per workgroup
    launch_score<F32, 4, 2, 2, 2>(q, q_stride, keys, N, H, NK, half, s1, s2, stream);
}

}  // namespace
}  // namespace smlm

extern "C" int smlm_pkm_score(const void *q, int64_t q_row_stride, const void *keys, int dtype, int64_t N, int H,
                              int NK, int half, void *s1, void *s2, void *stream) {
  using namespace smlm;
  if (!q || !keys || !s1 || !s2) return fail(SMLM_EINVAL, "smlm_pkm_score: null q, keys, s1 or s2 pointer");
  if (dtype != SMLM_BF16 && dtype != SMLM_F32)
    return fail(SMLM_EINVAL, "smlm_pkm_score: dtype must be SMLM_BF16 or SMLM_F32, got %d", dtype);
  if (N < 0 || N > 0x7FFFFFFFLL || H < 1 || H > 32768 || NK < 1 || half < 1)
    return fail(SMLM_EINVAL, "smlm_pkm_score: bad shape N=%lld H=%d NK=%d half=%d", (long long)N, H, NK, half);
  const int epl = dtype == SMLM_F32 ? 4 : 8;
  if (half % epl)
    return fail(SMLM_EUNSUPPORTED, "smlm_pkm_score: half=%d must be a multiple of %d for this dtype", half, epl);
  if (q_row_stride < 2LL * H * half || q_row_stride % epl)
    return fail(SMLM_EINVAL, "smlm_pkm_score: q_row_stride=%lld must be >= H*2*half and a multiple of %d",
                (long long)q_row_stride, epl);
  if (((uintptr_t)q | (uintptr_t)keys | (uintptr_t)s1 | (uintptr_t)s2) % 16)
    return fail(SMLM_EINVAL, "smlm_pkm_score: q, keys, s1 and s2 must be 16-byte aligned");
  if (N == 0) return SMLM_OK;
  if (dtype == SMLM_F32) dispatch_score<true>(q, q_row_stride, keys, N, H, NK, half, s1, s2, (hipStream_t)stream);
  else dispatch_score<false>(q, q_row_stride, keys, N, H, NK, half, s1, s2, (hipStream_t)stream);
  return launch_status("smlm_pkm_score");
}
