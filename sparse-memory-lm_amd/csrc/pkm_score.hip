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
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

// 16 bytes at p (always a valid address: callers clamp row indices into range), or zeros if !ok.  Selecting the
// loaded value rather than the address keeps the load a plain global load (a select between a global pointer and
// a local zero turns it into a flat load with the zero in scratch memory).
__device__ __forceinline__ uint4 load16_or_zero(const void *p, bool ok) {
  const uint4 v = *(const uint4 *)p;
  return ok ? v : uint4{0u, 0u, 0u, 0u};
}

// One k-step's operand fragments of score_kernel: key rows key0 + 16 i + r and token rows tok0 + 16 j + r, the
// g-th group of EPL dims from k0 (zeros outside the rows or past half).
template <int ESZ, int EPL, int WM, int WN>
__device__ __forceinline__ void score_load_step(const char *kbase, const char *qbase, int64_t q_stride, int N, int NK,
                                                int half, int key0, int tok0, int r, int g, int k0, u32x4 (&a)[WM],
                                                u32x4 (&b)[WN]) {
  const int kk = k0 + g * EPL;
  const bool kin = kk < half;  // half % EPL == 0: a lane's group is entirely inside or outside
#pragma unroll
  for (int i = 0; i < WM; ++i) {
    const int key = key0 + i * 16 + r;
    a[i] = __builtin_bit_cast(u32x4, load16_or_zero(kbase + ((int64_t)min(key, NK - 1) * half + (kin ? kk : 0)) * ESZ,
                                                     kin && key < NK));
  }
#pragma unroll
  for (int j = 0; j < WN; ++j) {
    const int tok = tok0 + j * 16 + r;
    b[j] = __builtin_bit_cast(u32x4, load16_or_zero(qbase + ((int64_t)min(tok, N - 1) * q_stride + (kin ? kk : 0)) * ESZ,
                                                     kin && tok < N));
  }
}

// PRE > 0 (bf16 only): when half <= 32 * PRE, every operand fragment of the workgroup is loaded before the first
// product (decode sizes are latency-bound: one round trip instead of one per k-step).
template <bool F32, int WM, int WN, int WAVES_M, int WAVES_N, int PRE = 0>
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

  if constexpr (!F32 && PRE > 0) {
    if (half <= PRE * KSTEP) {
      uint4 a[PRE][WM], b[PRE][WN];
#pragma unroll
      for (int st = 0; st < PRE; ++st) {
        if (st * KSTEP >= half) continue;  // workgroup-uniform
        const int kk = st * KSTEP + g * EPL;
        const bool kin = kk < half;
#pragma unroll
        for (int i = 0; i < WM; ++i) {
          const int key = key0 + i * 16 + r;
          a[st][i] = load16_or_zero(kbase + ((int64_t)min(key, NK - 1) * half + (kin ? kk : 0)) * ESZ,
                                    kin && key < NK);
        }
#pragma unroll
        for (int j = 0; j < WN; ++j) {
          const int tok = tok0 + j * 16 + r;
          b[st][j] = load16_or_zero(qbase + ((int64_t)min(tok, N - 1) * q_stride + (kin ? kk : 0)) * ESZ,
                                    kin && tok < N);
        }
      }
#pragma unroll
      for (int st = 0; st < PRE; ++st) {
        if (st * KSTEP >= half) continue;
#pragma unroll
        for (int i = 0; i < WM; ++i)
#pragma unroll
          for (int j = 0; j < WN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a[st][i]),
                                                                __builtin_bit_cast(bf16x8, b[st][j]), acc[i][j], 0, 0,
                                                                0);
      }
    }
  }
  // Operands of step k0 + KSTEP are in flight while the MFMAs of step k0 run.  fp32: the four products of a
  // 16-byte group are issued group-slot outer, so consecutive MFMAs feed different accumulators; each
  // accumulator still adds its products in the same order (slot 0..3 of step 0, of step 1, ...).
  const int kbeg = (!F32 && PRE > 0 && half <= PRE * KSTEP) ? half : 0;
  u32x4 a[WM], b[WN];
  if (kbeg < half)
    score_load_step<ESZ, EPL, WM, WN>(kbase, qbase, q_stride, N, NK, half, key0, tok0, r, g, kbeg, a, b);
  for (int k0 = kbeg; k0 < half; k0 += KSTEP) {
    const bool more = k0 + KSTEP < half;  // workgroup-uniform
    u32x4 an[WM], bn[WN];
    if (more)
      score_load_step<ESZ, EPL, WM, WN>(kbase, qbase, q_stride, N, NK, half, key0, tok0, r, g, k0 + KSTEP, an, bn);
    if constexpr (F32) {
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int i = 0; i < WM; ++i)
#pragma unroll
          for (int j = 0; j < WN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(__builtin_bit_cast(floatx4, a[i])[s],
                                                             __builtin_bit_cast(floatx4, b[j])[s], acc[i][j], 0, 0,
                                                             0);
    } else {
#pragma unroll
      for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < WN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a[i]),
                                                              __builtin_bit_cast(bf16x8, b[j]), acc[i][j], 0, 0, 0);
    }
    if (more) {
#pragma unroll
      for (int i = 0; i < WM; ++i) a[i] = an[i];
#pragma unroll
      for (int j = 0; j < WN; ++j) b[j] = bn[j];
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
    const int kc = kin ? kk : 0;                                                                            \
    a0 = load16_or_zero(kbase + (int64_t)min(key0 + pr0, NK - 1) * half + kc, kin && key0 + pr0 < NK);     \
    a1 = load16_or_zero(kbase + (int64_t)min(key0 + pr1, NK - 1) * half + kc, kin && key0 + pr1 < NK);     \
    b0 = load16_or_zero(qbase + (int64_t)min(tok0 + pr0, N - 1) * q_stride + kc, kin && tok0 + pr0 < N);   \
    b1 = load16_or_zero(qbase + (int64_t)min(tok0 + pr1, N - 1) * q_stride + kc, kin && tok0 + pr1 < N);   \
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

// bf16, many tokens: query-stationary streaming.  A workgroup = 4 wavefronts = 256 tokens of one (head, half).
// Wavefront w keeps the query fragments of its 64 tokens for the whole contraction in registers (half / 32 steps x
// 4 token tiles), and the workgroup streams the sub-keys through LDS in blocks of 64 rows, double-buffered: while
// the 16 x (half / 32) MFMAs of block b run, block b + 1 is in flight from memory into registers, written to the
// other LDS buffer afterwards (one barrier per block).  Every A fragment read from LDS feeds 4 MFMAs (LDS traffic
// half of its bandwidth at full MFMA rate), and the 64 x 64 scores of a block go straight from the accumulators to
// memory (4 consecutive sub-keys = one 8-byte store per lane).  LDS rows are padded by 16 bytes so that the 16 rows
// one fragment read touches fall on distinct banks.  1-D grid: workgroup i serves (head, half) z = i % 2H and runs
// on XCD i % 8, so with 2H dividing 8 every XCD reads one sub-key set only (1 MB at NK 2048) and keeps it in its L2.
// The sums run over the 32-dim steps in the same order as score_lds_kernel, so the bits are the same.
constexpr int kStreamKeys = 64;     // sub-keys per streamed block
constexpr int kStreamWaveTok = 64;  // tokens per wavefront


template <int KSTEPS, int WAVES>
__global__ void __launch_bounds__(WAVES * 64)
    score_stream_kernel(const uint16_t *__restrict__ q, int64_t q_stride, const uint16_t *__restrict__ keys, int N,
                        int H, int NK, uint16_t *__restrict__ s1, uint16_t *__restrict__ s2) {
  constexpr int NT = WAVES * 64;            // threads
  constexpr int HALF = KSTEPS * 32;
  constexpr int RS = HALF + 8;              // LDS row stride (bf16)
  constexpr int PPR = HALF / 8;             // 16-byte pieces per sub-key row
  constexpr int PPT = kStreamKeys * PPR / NT;   // pieces per thread per block
  constexpr int ROWS_PER_PASS = NT / PPR;
  static_assert(PPT >= 1 && kStreamKeys * PPR % NT == 0, "block pieces must split evenly over the threads");
  __shared__ __align__(16) uint16_t sA[2][kStreamKeys * RS];
  const int Z = 2 * H;
  const int z = (int)(blockIdx.x % Z), tile = (int)(blockIdx.x / Z);
  const int h = z >> 1, p = z & 1;
  const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
  const int r = lane & 15, g = lane >> 4;
  const int tok0 = tile * (WAVES * kStreamWaveTok) + wave * kStreamWaveTok;
  const uint16_t *kbase = keys + (int64_t)z * NK * HALF;
  const uint16_t *qbase = q + (int64_t)h * 2 * HALF + (int64_t)p * HALF;
  uint16_t *out = p ? s2 : s1;
  const bool all_tok = tok0 + kStreamWaveTok <= N;   // wavefront-uniform: no token guards needed

  bf16x8 bq[4][KSTEPS];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int tok = tok0 + j * 16 + r;
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s)
      bq[j][s] = __builtin_bit_cast(
          bf16x8, load16_or_zero(qbase + (int64_t)min(tok, N - 1) * q_stride + s * 32 + g * 8, tok < N));
  }

  // this thread's pieces of a block: rows prow + ROWS_PER_PASS * i, 16-byte column pcol
  const int prow = tid / PPR, pcol = (tid % PPR) * 8;
  const int nkb = (NK + kStreamKeys - 1) / kStreamKeys;
  const int nfull = NK / kStreamKeys;       // blocks with all 64 sub-keys present
  uint4 stage[PPT];
#define SMLM_STREAM_FETCH(kb)                                                                                    \
  if ((kb) < nfull) {                                                                                           \
    const uint16_t *src = kbase + ((int64_t)(kb) * kStreamKeys + prow) * HALF + pcol;                          \
    _Pragma("unroll") for (int i = 0; i < PPT; ++i) stage[i] = *(const uint4 *)(src + ROWS_PER_PASS * i * HALF); \
  } else {                                                                                                      \
    _Pragma("unroll") for (int i = 0; i < PPT; ++i) {                                                           \
      const int key = (kb) * kStreamKeys + prow + ROWS_PER_PASS * i;                                            \
      stage[i] = load16_or_zero(kbase + (int64_t)min(key, NK - 1) * HALF + pcol, key < NK);                    \
    }                                                                                                           \
  }
#define SMLM_STREAM_PUT(buf)                                                                                     \
  _Pragma("unroll") for (int i = 0; i < PPT; ++i)                                                               \
      *(uint4 *)&sA[(buf)][(prow + ROWS_PER_PASS * i) * RS + pcol] = stage[i];

  SMLM_STREAM_FETCH(0)
  SMLM_STREAM_PUT(0)
  __syncthreads();
  for (int kb = 0; kb < nkb; ++kb) {
    // 1. the next block in flight; 2. this block's products; 3. the next block into the other buffer;
    // 4. this block's scores out (their stores drain during the next block's products)
    if (kb + 1 < nkb) {
      SMLM_STREAM_FETCH(kb + 1)
    }
    const uint16_t *A = sA[kb & 1];
    floatx4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) {
      bf16x8 a[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = *(const bf16x8 *)&A[(i * 16 + r) * RS + s * 32 + g * 8];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], bq[j][s], acc[i][j], 0, 0, 0);
    }
    if (kb + 1 < nkb) {
      SMLM_STREAM_PUT((kb + 1) & 1)
    }
    const int key0 = kb * kStreamKeys + g * 4;
    if (all_tok && kb < nfull) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint16_t *orow = out + ((int64_t)(tok0 + j * 16 + r) * H + h) * NK + key0;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          *(uint2 *)(orow + i * 16) = uint2{pack_bf16x2(acc[i][j][0], acc[i][j][1]),
                                            pack_bf16x2(acc[i][j][2], acc[i][j][3])};
      }
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int tok = tok0 + j * 16 + r;
        uint16_t *orow = out + ((int64_t)tok * H + h) * NK + key0;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (tok < N && key0 + i * 16 < NK)
            *(uint2 *)(orow + i * 16) = uint2{pack_bf16x2(acc[i][j][0], acc[i][j][1]),
                                              pack_bf16x2(acc[i][j][2], acc[i][j][3])};
      }
    }
    __syncthreads();
  }
#undef SMLM_STREAM_FETCH
#undef SMLM_STREAM_PUT
}

// bf16, many tokens, NK % 64 == 0: the query-stationary stream with the wavefronts specialised.  A workgroup = 4
// compute wavefronts (64 tokens each, query fragments in registers for the whole launch) + 4 memory wavefronts, 256
// tokens of one (head, half).  Per 64-sub-key block kb the compute wavefronts run the MFMAs on LDS block kb and write
// their bf16 scores to an LDS output tile; meanwhile the memory wavefronts put block kb + 1 (fetched during the
// previous block) into the other LDS key buffer, fetch block kb + 2, and write block kb - 1's output tile to memory
// as whole 128-byte score rows.  A wavefront that stalls on a store is then never one that has MFMAs to issue: the
// stores (537 MB at config 2) and the products overlap.  One barrier per block.  The score rows are written with
// non-temporal stores: they stream to memory instead of displacing the caches (0.217 -> 0.148 ms at config 2).
// The key rows in LDS are padded by 32 bytes (the compute wavefronts' fragment reads conflict less than with 16).
constexpr int kWsTok = 256;             // tokens per workgroup
constexpr int kWsOutStride = kStreamKeys + 8;  // LDS output tile row stride (bf16)

template <int KSTEPS>
__global__ void __launch_bounds__(512)
    score_ws_kernel(const uint16_t *__restrict__ q, int64_t q_stride, const uint16_t *__restrict__ keys, int N,
                    int H, int NK, uint16_t *__restrict__ s1, uint16_t *__restrict__ s2) {
  constexpr int HALF = KSTEPS * 32;
  // LDS key row stride (bf16): rows padded by 32 bytes.  Measured with SQ_LDS_BANK_CONFLICT at config 2: 14.7 M
  // conflict cycles per launch with 16 bytes of padding (and with 48), 6.3 M with 32; 139-140 -> 135.5-136 us.  The
  // output tile's share: unpadded rows with the 16-byte pieces XOR-swizzled by row took the count to 4.2 M and the
  // time nowhere (135-137 us); wider padding raised it (16.8-25.2 M), no padding at all 62.9 M (234 us)
  constexpr int RS = HALF + 16;
  constexpr int PPR = HALF / 8;              // 16-byte pieces per sub-key row
  constexpr int PPT = kStreamKeys * PPR / 256;   // key pieces per memory thread per block
  constexpr int RPP = 256 / PPR;             // key rows per memory pass
  constexpr int OPT = kWsTok * kStreamKeys / 8 / 256;  // 16-byte output pieces per memory thread per block (8)
  __shared__ __align__(16) uint16_t sA[2 * kStreamKeys * RS];          // 2 key blocks of 64 rows
  __shared__ __align__(16) uint16_t sO[2 * kWsTok * kWsOutStride];     // 2 output tiles of 256 token rows
  const int Z = 2 * H;
  const int z = (int)(blockIdx.x % Z), tile = (int)(blockIdx.x / Z);
  const int h = z >> 1, p = z & 1;
  const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
  const uint16_t *kbase = keys + (int64_t)z * NK * HALF;
  uint16_t *out = p ? s2 : s1;
  const int tok_base = tile * kWsTok;
  const int nkb = NK / kStreamKeys;

  if (wave < 4) {
    // ---- compute wavefronts
    const int r = lane & 15, g = lane >> 4;
    const int tok0 = tok_base + wave * kStreamWaveTok;
    const uint16_t *qbase = q + (int64_t)h * 2 * HALF + (int64_t)p * HALF;
    bf16x8 bq[4][KSTEPS];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int tok = tok0 + j * 16 + r;
#pragma unroll
      for (int s = 0; s < KSTEPS; ++s)
        bq[j][s] = __builtin_bit_cast(
            bf16x8, load16_or_zero(qbase + (int64_t)min(tok, N - 1) * q_stride + s * 32 + g * 8, tok < N));
    }
    __syncthreads();  // block 0 is in sA[0]
    for (int kb = 0; kb < nkb; ++kb) {
      const uint16_t *A = sA + (kb & 1) * kStreamKeys * RS;
      floatx4 acc[4][4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KSTEPS; ++s) {
        bf16x8 a[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) a[i] = *(const bf16x8 *)&A[(i * 16 + r) * RS + s * 32 + g * 8];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], bq[j][s], acc[i][j], 0, 0, 0);
      }
      // lane (r, g) holds keys 16 i + 4 g .. +3 of token 16 j + r: into the output tile
      uint16_t *O = sO + (kb & 1) * kWsTok * kWsOutStride + (wave * kStreamWaveTok) * kWsOutStride;
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          *(uint2 *)&O[(j * 16 + r) * kWsOutStride + i * 16 + g * 4] =
              uint2{pack_bf16x2(acc[i][j][0], acc[i][j][1]), pack_bf16x2(acc[i][j][2], acc[i][j][3])};
      __syncthreads();
    }
    // done: the memory wavefronts write the last tile after the last barrier (1 + nkb barriers on both sides)
  } else {
    // ---- memory wavefronts: thread mt = 0..255
    const int mt = tid - 256;
    const int prow = mt / PPR, pcol = (mt % PPR) * 8;
    u32x4 stage[PPT];  // a native vector type: an array of it stays in registers
    // block 0 into sA[0], block 1 into registers
#pragma unroll
    for (int i = 0; i < PPT; ++i)
      stage[i] = *(const u32x4 *)(kbase + ((int64_t)prow + RPP * i) * HALF + pcol);
#pragma unroll
    for (int i = 0; i < PPT; ++i) *(u32x4 *)&sA[(prow + RPP * i) * RS + pcol] = stage[i];
    if (nkb > 1) {
#pragma unroll
      for (int i = 0; i < PPT; ++i)
        stage[i] = *(const u32x4 *)(kbase + ((int64_t)kStreamKeys + prow + RPP * i) * HALF + pcol);
    }
    __syncthreads();
    for (int kb = 0; kb <= nkb; ++kb) {
      if (kb + 1 < nkb) {  // block kb + 1 into the other key buffer (its last readers finished block kb - 1)
        uint16_t *A = sA + ((kb + 1) & 1) * kStreamKeys * RS;
#pragma unroll
        for (int i = 0; i < PPT; ++i) *(u32x4 *)&A[(prow + RPP * i) * RS + pcol] = stage[i];
      }
      if (kb + 2 < nkb) {
        const uint16_t *src = kbase + ((int64_t)(kb + 2) * kStreamKeys + prow) * HALF + pcol;
#pragma unroll
        for (int i = 0; i < PPT; ++i) stage[i] = *(const u32x4 *)(src + (int64_t)RPP * i * HALF);
      }
      if (kb >= 1) {  // block kb - 1's scores: rows of 64 sub-keys = 8 pieces of 16 bytes
        const uint16_t *O = sO + ((kb - 1) & 1) * kWsTok * kWsOutStride;
        const int key0 = (kb - 1) * kStreamKeys;
#pragma unroll
        for (int u = 0; u < OPT; ++u) {
          const int id = mt + 256 * u, t = id >> 3, c = id & 7;
          const u32x4 v = *(const u32x4 *)&O[t * kWsOutStride + c * 8];
          const int tok = tok_base + t;
          if (tok < N) __builtin_nontemporal_store(v, (u32x4 *)(out + ((int64_t)tok * H + h) * NK + key0 + c * 8));
        }
      }
      if (kb < nkb) __syncthreads();
    }
  }
}

// bf16 decode sizes (N <= 64, half <= 256): a workgroup = 4 wavefronts x 32 sub-keys = 128 sub-keys against 16 * MT
// tokens.  The query tile is loaded once per workgroup into LDS (the four wavefronts share it), each wavefront's
// sub-key rows go straight into registers, and every load is issued before the first product.
template <int MT, int KT = 1>
__global__ void __launch_bounds__(256)
    score_decode_kernel(const uint16_t *__restrict__ q, int64_t q_stride, const uint16_t *__restrict__ keys, int N,
                        int H, int NK, int half, uint16_t *__restrict__ s1, uint16_t *__restrict__ s2) {
  constexpr int MAXST = 8;                 // k-steps of 32 (half <= 256)
  constexpr int RS = MAXST * 32 + 8;       // LDS row stride (bf16)
  __shared__ __align__(16) uint16_t sQ[16 * MT * RS];
  const int z = blockIdx.z, h = z >> 1, p = z & 1;
  const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64, r = lane & 15, g = lane >> 4;
  const int key0 = blockIdx.x * (64 * KT) + wave * (16 * KT);   // KT 16-key tiles per wavefront
  const int tok0 = blockIdx.y * (16 * MT);
  const uint16_t *kbase = keys + (int64_t)z * NK * half;
  const uint16_t *qbase = q + (int64_t)h * 2 * half + (int64_t)p * half;
  const int nst = (half + 31) / 32;

  // 1. this wavefront's sub-key fragments (steps past half and keys past NK load valid memory, then zero)
  uint4 a[MAXST][KT];
#pragma unroll
  for (int st = 0; st < MAXST; ++st) {
    if (st >= nst) continue;  // workgroup-uniform
    const int kk = st * 32 + g * 8;
    const bool kin = kk < half;
#pragma unroll
    for (int i = 0; i < KT; ++i) {
      const int key = key0 + i * 16 + r;
      a[st][i] = load16_or_zero(kbase + (int64_t)min(key, NK - 1) * half + (kin ? kk : 0), kin && key < NK);
    }
  }
  // 2. the query tile into LDS: row t (token tok0 + t), 16-byte chunks c < half / 8; tokens past N are zero rows
  const int cpr = half / 8, chunks = 16 * MT * cpr;
  constexpr int kMaxChunks = 16 * MT * MAXST * 4;
  uint4 qv[(kMaxChunks + 255) / 256];
#pragma unroll
  for (int u = 0; u < (kMaxChunks + 255) / 256; ++u) {
    const int ch = tid + u * 256;
    if (ch >= chunks) continue;
    const int t = ch / cpr, c = ch % cpr;
    qv[u] = load16_or_zero(qbase + (int64_t)min(tok0 + t, N - 1) * q_stride + c * 8, tok0 + t < N);
  }
#pragma unroll
  for (int u = 0; u < (kMaxChunks + 255) / 256; ++u) {
    const int ch = tid + u * 256;
    if (ch >= chunks) continue;
    const int t = ch / cpr, c = ch % cpr;
    *(uint4 *)&sQ[t * RS + c * 8] = qv[u];
  }
  // the steps' k groups past half read columns [half, 32 * nst) of the tile: zero them
  for (int i = tid; i < 16 * MT * (nst * 4 - cpr); i += 256) {
    const int t = i / (nst * 4 - cpr), c = cpr + i % (nst * 4 - cpr);
    *(uint4 *)&sQ[t * RS + c * 8] = uint4{0u, 0u, 0u, 0u};
  }
  __syncthreads();

  // 3. products
  floatx4 acc[KT][MT];
#pragma unroll
  for (int i = 0; i < KT; ++i)
#pragma unroll
    for (int j = 0; j < MT; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int st = 0; st < MAXST; ++st) {
    if (st >= nst) continue;
#pragma unroll
    for (int j = 0; j < MT; ++j) {
      const uint4 b = *(const uint4 *)&sQ[(j * 16 + r) * RS + st * 32 + g * 8];
#pragma unroll
      for (int i = 0; i < KT; ++i)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a[st][i]),
                                                            __builtin_bit_cast(bf16x8, b), acc[i][j], 0, 0, 0);
    }
  }

  // 4. scores: lane (r, g) holds sub-keys key0 + 16 i + 4g .. +3 of token tok0 + 16 j + r
  uint16_t *out = p ? s2 : s1;
#pragma unroll
  for (int i = 0; i < KT; ++i)
#pragma unroll
    for (int j = 0; j < MT; ++j) {
      const int tok = tok0 + j * 16 + r;
      const int key = key0 + i * 16 + g * 4;
      if (tok >= N || key >= NK) continue;
      uint16_t *o = out + ((int64_t)tok * H + h) * NK + key;
      const floatx4 v = acc[i][j];
      if ((NK & 3) == 0) {  // key % 4 == 0 and NK % 4 == 0: the 4 scores are in range and 8-byte aligned
        *(uint2 *)o = uint2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (key + e < NK) o[e] = (uint16_t)bf16_bits_rtne(v[e]);
      }
    }
}

template <bool F32, int WM, int WN, int WAVES_M, int WAVES_N, int PRE = 0>
void launch_score(const void *q, int64_t q_stride, const void *keys, int64_t N, int H, int NK, int half, void *s1,
                  void *s2, hipStream_t stream) {
  constexpr int BM = WAVES_M * WM * 16, BN = WAVES_N * WN * 16;
  const dim3 grid((unsigned)((N + BN - 1) / BN), (unsigned)((NK + BM - 1) / BM), (unsigned)(2 * H));
  hipLaunchKernelGGL((score_kernel<F32, WM, WN, WAVES_M, WAVES_N, PRE>), grid, dim3(WAVES_M * WAVES_N * 64), 0,
                     stream, q, q_stride, keys, (int)N, H, NK, half, s1, s2);
}

template <bool F32>
void dispatch_score(const void *q, int64_t q_stride, const void *keys, int64_t N, int H, int NK, int half, void *s1,
                    void *s2, hipStream_t stream) {
  if (!F32 && N <= 64 && half <= 256) {  // decode: 128 sub-keys x 16 or 64 tokens, query tile shared in LDS
    // 64 sub-keys per workgroup (one 16-key tile per wavefront): 512 workgroups at 4,096 sub-keys per half, each
    // CU pulling 32 KB of sub-keys
    const int kb = 64;
    const dim3 grid((unsigned)((NK + kb - 1) / kb), (unsigned)((N + (N <= 16 ? 15 : 63)) / (N <= 16 ? 16 : 64)),
                    (unsigned)(2 * H));  // x: sub-key blocks, y: token blocks, z: (head, half)
    if (N <= 16)
      hipLaunchKernelGGL((score_decode_kernel<1, 1>), grid, dim3(256), 0, stream, (const uint16_t *)q, q_stride,
                         (const uint16_t *)keys, (int)N, H, NK, half, (uint16_t *)s1, (uint16_t *)s2);
    else
      hipLaunchKernelGGL((score_decode_kernel<4, 1>), grid, dim3(256), 0, stream, (const uint16_t *)q, q_stride,
                         (const uint16_t *)keys, (int)N, H, NK, half, (uint16_t *)s1, (uint16_t *)s2);
  } else if (N <= 16) {  // (fp32 or half > 256) decode: 128 sub-keys x 16 tokens per workgroup
    launch_score<F32, 2, 1, 4, 1, F32 ? 0 : 8>(q, q_stride, keys, N, H, NK, half, s1, s2, stream);
  } else if (!F32 && N <= 64) {  // decode batches: 128 sub-keys x 64 tokens, operands preloaded
    launch_score<F32, 4, 2, 2, 2, F32 ? 0 : 8>(q, q_stride, keys, N, H, NK, half, s1, s2, stream);
  } else if (F32 || (N / 128 + 1) * (NK / 128 + 1) * 2 * (int64_t)H >= (1LL << 30)) {
    // 256 sub-keys x 64 tokens per workgroup (8 x 2 tiles per wavefront: each 16-byte operand feeds 6.4 MFMAs;
    // config-0 fp32 scoring 132 -> 108 us against 4 x 2), operands straight from memory
    launch_score<F32, 8, 2, 2, 2>(q, q_stride, keys, N, H, NK, half, s1, s2, stream);
  } else if (!F32 && (half == 64 || half == 128 || half == 256) && NK % 4 == 0 && N >= 256 &&
             (N + 255) / 256 * 2 * (int64_t)H >= 256) {  // enough 256-token tiles to give every CU one
    // bf16, many tokens: query-stationary streaming of the sub-keys
    const int64_t tiles = (N + 255) / 256;
    const dim3 grid((unsigned)(tiles * 2 * H));
    if (NK % kStreamKeys == 0) {  // whole blocks: compute and memory wavefronts specialised
#define SMLM_WS(KS)                                                                                           \
  hipLaunchKernelGGL((score_ws_kernel<KS>), grid, dim3(512), 0, stream, (const uint16_t *)q, q_stride,        \
                     (const uint16_t *)keys, (int)N, H, NK, (uint16_t *)s1, (uint16_t *)s2)
      if (half == 256) SMLM_WS(8);
      else if (half == 128) SMLM_WS(4);
      else SMLM_WS(2);
#undef SMLM_WS
      return;
    }
#define SMLM_STREAM(KS)                                                                                       \
  hipLaunchKernelGGL((score_stream_kernel<KS, 4>), grid, dim3(256), 0, stream, (const uint16_t *)q, q_stride,  \
                     (const uint16_t *)keys, (int)N, H, NK, (uint16_t *)s1, (uint16_t *)s2)
    if (half == 256) SMLM_STREAM(8);
    else if (half == 128) SMLM_STREAM(4);
    else SMLM_STREAM(2);
#undef SMLM_STREAM
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
