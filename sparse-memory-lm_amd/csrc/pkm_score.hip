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
          const floatx4 fa = __builtin_bit_cast(floatx4, a[i]);
          const floatx4 fb = __builtin_bit_cast(floatx4, b[j]);
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
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if (key + e >= NK) continue;
          if constexpr (F32) ((float *)out)[o + e] = v[e];
          else ((uint16_t *)out)[o + e] = (uint16_t)bf16_bits_rtne(v[e]);
        }
      }
    }
}

// bf16, many tokens: 128 sub-keys x 128 tokens per workgroup (2 x 2 wavefronts of 64 x 64).  The contraction
// runs in chunks of 32 dims through two LDS stages: while the MFMAs consume one stage, the next chunk is already
// in flight from memory into registers (two 16-byte pieces of each operand per thread) and is written to the
// other stage afterwards, so one barrier per chunk separates them.  LDS rows are padded to 40 bf16 (80 B) so the
// 16 rows a fragment read touches fall on distinct banks.

template <int WM, int WN>
__global__ void __launch_bounds__(256)
    score_lds_kernel(const uint16_t *__restrict__ q, int64_t q_stride, const uint16_t *__restrict__ keys, int N,
                     int H, int NK, int half, uint16_t *__restrict__ s1, uint16_t *__restrict__ s2) {
  constexpr int BM = 2 * 16 * WM, BN = 2 * 16 * WN;
  constexpr int KC = 32, RS = KC + 8, PR = KC / 8;   // dims per chunk, LDS row stride, 16-byte pieces per row
  __shared__ __align__(16) uint16_t sAB[2 * (BM + BN) * RS];
  // 1-D grid, XCD-aware: workgroup b runs on XCD b % 8, so tile t = (b % 8) * per_xcd + b / 8 gives each XCD a
  // contiguous run of tiles; tiles are ordered sub-key tile fastest, so an XCD's L2 reads each token tile's
  // queries once and reuses them for all sub-key tiles of that (head, half).
  const int key_tiles = (NK + BM - 1) / BM, tok_tiles = (N + BN - 1) / BN;
  const int per_xcd = gridDim.x / 8;
  const int t = (int)(blockIdx.x % 8) * per_xcd + (int)(blockIdx.x / 8);
  if (t >= key_tiles * tok_tiles * 2 * H) return;
  const int z = t / (key_tiles * tok_tiles);
  const int h = z >> 1, p = z & 1;
  const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
  const int wm = wave & 1, wn = wave >> 1;
  const int r = lane & 15, g = lane >> 4;
  const int key0 = (t % key_tiles) * BM, tok0 = ((t / key_tiles) % tok_tiles) * BN;
  const uint16_t *kbase = keys + (int64_t)(h * 2 + p) * NK * half;
  const uint16_t *qbase = q + (int64_t)h * 2 * half + (int64_t)p * half;
  const uint4 zero = {0u, 0u, 0u, 0u};

  floatx4 acc[WM][WN];
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int j = 0; j < WN; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  static_assert(BM * PR == 512 && BN * PR == 512, "two pieces per thread per operand");
  // thread -> (row, piece) for its two A and two B pieces
  const int pr0 = tid / PR, pc0 = (tid % PR) * 8, pr1 = pr0 + 64;
  uint4 a0, a1, b0, b1;
#define SMLM_FETCH(k0)                                                                                      \
  {                                                                                                         \
    const int kk = (k0) + pc0;                                                                              \
    const bool kin = kk < half;                                                                             \
    a0 = (kin && key0 + pr0 < NK) ? *(const uint4 *)(kbase + (int64_t)(key0 + pr0) * half + kk) : zero;    \
    a1 = (kin && key0 + pr1 < NK) ? *(const uint4 *)(kbase + (int64_t)(key0 + pr1) * half + kk) : zero;    \
    b0 = (kin && tok0 + pr0 < N) ? *(const uint4 *)(qbase + (int64_t)(tok0 + pr0) * q_stride + kk) : zero; \
    b1 = (kin && tok0 + pr1 < N) ? *(const uint4 *)(qbase + (int64_t)(tok0 + pr1) * q_stride + kk) : zero; \
  }
#define SMLM_STAGE(s)                                                                                       \
  {                                                                                                         \
    uint16_t *sa = sAB + (s) * (BM + BN) * RS, *sb = sa + BM * RS;                                          \
    *(uint4 *)&sa[pr0 * RS + pc0] = a0;                                                                     \
    *(uint4 *)&sa[pr1 * RS + pc0] = a1;                                                                     \
    *(uint4 *)&sb[pr0 * RS + pc0] = b0;                                                                     \
    *(uint4 *)&sb[pr1 * RS + pc0] = b1;                                                                     \
  }
  SMLM_FETCH(0)
  SMLM_STAGE(0)
  const int nck = (half + KC - 1) / KC;
  for (int c = 0; c < nck; ++c) {
    if (c + 1 < nck) SMLM_FETCH((c + 1) * KC)
    __syncthreads();
    const uint16_t *sa = sAB + (c & 1) * (BM + BN) * RS, *sb = sa + BM * RS;
    bf16x8 fa[WM], fb[WN];
#pragma unroll
    for (int i = 0; i < WM; ++i) fa[i] = *(const bf16x8 *)&sa[(wm * 16 * WM + i * 16 + r) * RS + g * 8];
#pragma unroll
    for (int j = 0; j < WN; ++j) fb[j] = *(const bf16x8 *)&sb[(wn * 16 * WN + j * 16 + r) * RS + g * 8];
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
      for (int j = 0; j < WN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
    if (c + 1 < nck) SMLM_STAGE((c + 1) & 1)
  }
#undef SMLM_FETCH
#undef SMLM_STAGE

  // Epilogue through LDS: the bf16 tile is written as [token][sub-key] rows (padded to kOutRS), then stored with
  // 16-byte loads per lane covering whole 256-byte token rows of the output.
  constexpr int kOutRS = BM + 8;

  static_assert(BN * kOutRS <= 2 * (BM + BN) * RS, "output tile must fit in the operand LDS");
  uint16_t *sOut = sAB;
  __syncthreads();      // all fragment reads of the last chunk are done
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int j = 0; j < WN; ++j) {
      const floatx4 v = acc[i][j];
      uint2 pk;
      pk.x = bf16_bits_rtne(v[0]) | (bf16_bits_rtne(v[1]) << 16);
      pk.y = bf16_bits_rtne(v[2]) | (bf16_bits_rtne(v[3]) << 16);
      *(uint2 *)&sOut[(wn * 16 * WN + j * 16 + r) * kOutRS + wm * 16 * WM + i * 16 + g * 4] = pk;
    }
  __syncthreads();
  uint16_t *out = p ? s2 : s1;
  constexpr int PPT = BM / 8;  // 16-byte pieces per token row of the tile
#pragma unroll
  for (int k = 0; k < BN * PPT / 256; ++k) {
    const int piece = tid + 256 * k, tl = piece / PPT, kl = (piece % PPT) * 8;
    const int tok = tok0 + tl, key = key0 + kl;
    if (tok >= N || key >= NK) continue;
    const int64_t o = ((int64_t)tok * H + h) * NK + key;
    const uint4 v = *(const uint4 *)&sOut[tl * kOutRS + kl];
    if ((NK & 7) == 0) {
      *(uint4 *)(out + o) = v;
    } else {
      const uint16_t *e = (const uint16_t *)&v;
      for (int x = 0; x < 8; ++x)
        if (key + x < NK) out[o + x] = e[x];
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
  if (N <= 16) {  // decode: 128 sub-keys x 16 tokens per workgroup, spread over many workgroups
    launch_score<F32, 2, 1, 4, 1>(q, q_stride, keys, N, H, NK, half, s1, s2, stream);
  } else if (F32 || N <= 64 || (N / 128 + 1) * (NK / 128 + 1) * 2 * (int64_t)H >= (1LL << 30)) {
    // 128 sub-keys x 64 tokens per workgroup, operands straight from memory
    launch_score<F32, 4, 2, 2, 2>(q, q_stride, keys, N, H, NK, half, s1, s2, stream);
  } else {        // bf16, many tokens: LDS-staged 128 x 128 tiles
    constexpr int BM = 128, BN = 128;
    const int64_t tiles = ((NK + BM - 1) / BM) * ((N + BN - 1) / BN) * 2 * (int64_t)H;
    const dim3 grid((unsigned)(8 * ((tiles + 7) / 8)));  // a multiple of 8: every XCD gets the same count
    hipLaunchKernelGGL((score_lds_kernel<4, 4>), grid, dim3(256), 0, stream, (const uint16_t *)q, q_stride,
                       (const uint16_t *)keys, (int)N, H, NK, half, (uint16_t *)s1, (uint16_t *)s2);
  }
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
