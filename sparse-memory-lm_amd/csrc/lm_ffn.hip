// Prompt-pass projections on the matrix cores (v_mfma_f32_16x16x32_bf16, fp32 accumulation), bf16 activations x
// (M, K) and nn.Linear weights:
//   smlm_linear_swiglu: the FFN up-projection with the SwiGLU activation in its epilogue (smlm/model.py:110-118),
//     out[m, j] = bf16(bf16(silu(a)) * b), a = bf16(x[m] . w13[j]), b = bf16(x[m] . w13[hidden + j]): the roundings
//     of the w13 projection (bf16 output) followed by smlm_swiglu, in one launch that writes the (M, hidden)
//     activation only (the unfused pair writes and re-reads the (M, 2 hidden) projection);
//   smlm_prompt_linear: out = bf16(x W^T + bias) for the other projections of a prompt pass (wqkv, wo, w2, the
//     memory layer's swilu_proj and value_proj), where the library GEMMs' large tiles leave CUs idle.
//
// Workgroup = 4 wavefronts, a tile of 128 tokens x 128 weight rows.  SwiGLU: the 64 weight rows of a and the 64
// of b, so each lane's a and b accumulators hold the same (token, feature) pairs; wavefront w: tokens 64 (w & 1)
// .. +63, features 32 (w >> 1) .. +31 (4 MFMA weight tiles: a lo / hi, b lo / hi x 4 token tiles).  Plain: 128
// output features, wavefront w: tokens 64 (w & 1) .., features 64 (w >> 1) .. +63.  K is staged in
// LDS in chunks of 128 (rows padded by 32 bytes: the fragment reads of 16 rows then fall on distinct banks), the
// next chunk loaded into registers while the current one's products run.  The bf16 results go through LDS so that
// every output row piece is stored as whole 128 bytes.  1-D grid, XCD-aware: the feature blocks of one token tile
// run on one XCD (workgroup id % 8), so the tile's activation rows come from that XCD's L2.
//
// MFMA operand mapping (16x16x32, r = lane % 16, g = lane / 16): A = 16 weight rows x 32 k (lane: row r, k group
// g), B = 32 k x 16 tokens (lane: token r, k group g), D: lane holds features 4g..4g+3 of token r.
#include "pkm_common.h"

namespace smlm {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

constexpr int kFfnTok = 128;              // tokens per workgroup
constexpr int kFfnFeat = 64;              // output features per workgroup (+ their 64 b rows)
constexpr int kFfnKc = 128;               // K chunk staged in LDS
constexpr int kFfnRow = kFfnKc + 16;      // LDS row stride of a chunk (bf16)
constexpr int kFfnPieces = kFfnTok * kFfnKc / 8 / 256;  // 16-byte pieces per thread per operand per chunk (8)
constexpr int kXcds = 8;

// SWIGLU: the tile's 128 LDS weight rows are the a rows f0 .. f0 + 63 and the b rows hidden + f0 .. (64 output
// features); otherwise (plain projection, bf16 out) the rows f0 .. f0 + 127 (128 output features, N = hidden).
template <bool SWIGLU>
__global__ void __launch_bounds__(256)
    prompt_linear_kernel(const uint16_t *__restrict__ x, int64_t x_stride, const uint16_t *__restrict__ w,
                         int64_t w_stride, const uint16_t *__restrict__ bias, int64_t M, int K, int hidden,
                         uint16_t *__restrict__ out, int64_t out_stride) {
  constexpr int FEAT = SWIGLU ? kFfnFeat : 2 * kFfnFeat;       // output features per workgroup
  __shared__ __align__(16) uint16_t sW[2 * kFfnFeat * kFfnRow];  // 128 weight rows
  __shared__ __align__(16) uint16_t sX[kFfnTok * kFfnRow];       // token rows; later the output tile

  // tile: the feature blocks of token tile tt share an XCD
  const int nfb = hidden / FEAT;
  const int64_t ntt = (M + kFfnTok - 1) / kFfnTok;
  const int64_t id = blockIdx.x, xcd = id % kXcds, local = id / kXcds;
  const int64_t tt = xcd + kXcds * (local / nfb);
  const int fb = (int)(local % nfb);
  if (tt >= ntt) return;  // workgroup-uniform, before any barrier
  const int64_t t0 = tt * kFfnTok;
  const int f0 = fb * FEAT;

  const int tid = threadIdx.x, wave = tid / kWave, lane = lane_id();
  const int r = lane & 15, g = lane >> 4;
  const int th = wave & 1, fh = wave >> 1;

  // global -> registers: piece p = tid + 256 u of a chunk is row p / 16, 16-byte column p % 16 (16 consecutive
  // threads read one row's 256 bytes); rows past M re-read row M - 1 (their results are not stored).  Native
  // vector arrays, indexed at compile time, so that they stay in registers.
  u32x4 rw[kFfnPieces], rx[kFfnPieces];
#define SMLM_FFN_LOAD(K0)                                                                                      \
  _Pragma("unroll") for (int u = 0; u < kFfnPieces; ++u) {                                                     \
    const int p = tid + 256 * u, row = p / 16, c = p % 16;                                                     \
    const int64_t wrow = !SWIGLU ? (int64_t)f0 + row : row < kFfnFeat ? f0 + row : (int64_t)hidden + f0 + (row - kFfnFeat); \
    rw[u] = *(const u32x4 *)(w + wrow * w_stride + (K0) + c * 8);                                              \
    rx[u] = *(const u32x4 *)(x + min(t0 + row, M - 1) * x_stride + (K0) + c * 8);                             \
  }
#define SMLM_FFN_STORE()                                                                                       \
  _Pragma("unroll") for (int u = 0; u < kFfnPieces; ++u) {                                                     \
    const int p = tid + 256 * u, row = p / 16, c = p % 16;                                                     \
    *(u32x4 *)&sW[row * kFfnRow + c * 8] = rw[u];                                                              \
    *(u32x4 *)&sX[row * kFfnRow + c * 8] = rx[u];                                                              \
  }

  floatx4 acc[4][4];  // [weight tile: a lo, a hi, b lo, b hi][token tile]
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
  const int xbase = th * 64;  // this wavefront's LDS token rows; its weight rows of tile i: wrow_lds(i)
// SWIGLU: tiles a lo, a hi, b lo, b hi of features fh * 32 .. +31; otherwise 4 tiles of features fh * 64 .. +63
#define SMLM_FFN_WROW(i) (SWIGLU ? ((i) >> 1) * kFfnFeat + fh * 32 + ((i) & 1) * 16 : fh * 64 + (i) * 16)

  // the bias of the lane's output features (plain projection), loaded now: read in the epilogue it would add a
  // memory round trip after the products
  float bv[4][4] = {};
  if constexpr (!SWIGLU) {
    if (bias) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) bv[i][e] = bf16_bits_to_f32(bias[f0 + fh * 64 + i * 16 + 4 * g + e]);
    }
  }

  const int nchunks = K / kFfnKc;
  SMLM_FFN_LOAD(0)
  SMLM_FFN_STORE()
  __syncthreads();
  for (int ch = 0; ch < nchunks; ++ch) {
    if (ch + 1 < nchunks) {  // in flight during this chunk's products
      SMLM_FFN_LOAD((ch + 1) * kFfnKc)
    }
#pragma unroll
    for (int s = 0; s < kFfnKc / 32; ++s) {
      bf16x8 a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = *(const bf16x8 *)&sW[(SMLM_FFN_WROW(i) + r) * kFfnRow + s * 32 + g * 8];
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = *(const bf16x8 *)&sX[(xbase + j * 16 + r) * kFfnRow + s * 32 + g * 8];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    __syncthreads();  // every wavefront is done with this chunk
    if (ch + 1 < nchunks) {
      SMLM_FFN_STORE()
      __syncthreads();
    }
  }
#undef SMLM_FFN_LOAD
#undef SMLM_FFN_STORE
#undef SMLM_FFN_WROW

  // epilogue into the output tile in LDS (over the token rows, no longer read), then whole row pieces to memory.
  // SWIGLU: a, b rounded to bf16 as the projection's output, bf16(silu(a)) as smlm_swiglu, then bf16(s * b);
  // otherwise the projection plus its bias (fp32) rounded to bf16.
  uint16_t *sO = sX;
  constexpr int OROW = FEAT + 8;  // output tile row stride (bf16)
  if constexpr (SWIGLU) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint32_t o[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          uint32_t h[2];
#pragma unroll
          for (int q = 0; q < 2; ++q) {
            const float av = bf16_bits_to_f32(bf16_bits_rtne(acc[i][j][2 * e + q]));
            const float bv = bf16_bits_to_f32(bf16_bits_rtne(acc[2 + i][j][2 * e + q]));
            const float sv = round_bf16(av / (1.0f + expf(-av)));
            h[q] = bf16_bits_rtne(sv * bv);
          }
          o[e] = h[0] | (h[1] << 16);
        }
        const int tok = xbase + j * 16 + r, feat = fh * 32 + i * 16 + 4 * g;
        *(uint2 *)&sO[tok * OROW + feat] = uint2{o[0], o[1]};
      }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t lo = bf16_bits_rtne(acc[i][j][0] + bv[i][0]) | (bf16_bits_rtne(acc[i][j][1] + bv[i][1]) << 16);
        const uint32_t hi = bf16_bits_rtne(acc[i][j][2] + bv[i][2]) | (bf16_bits_rtne(acc[i][j][3] + bv[i][3]) << 16);
        const int tok = xbase + j * 16 + r, feat = fh * 64 + i * 16 + 4 * g;
        *(uint2 *)&sO[tok * OROW + feat] = uint2{lo, hi};
      }
  }
  __syncthreads();
  constexpr int PPR = FEAT / 8;   // 16-byte pieces per output row
#pragma unroll
  for (int u = 0; u < kFfnTok * PPR / 256; ++u) {
    const int p = tid + 256 * u, row = p / PPR, c = p % PPR;
    if (t0 + row < M)
      *(uint4 *)(out + (t0 + row) * out_stride + f0 + c * 8) = *(const uint4 *)&sO[row * OROW + c * 8];
  }
}

}  // namespace
}  // namespace smlm

namespace smlm {
namespace {

// shared checks and launch: N = the kernel's `hidden` (SWIGLU: the activation's width; otherwise the output width)
template <bool SWIGLU>
int launch_prompt_linear(const char *what, const void *x, int64_t x_row_stride, const void *w, int64_t w_row_stride,
                         const void *bias, int64_t M, int K, int N, void *out, int64_t out_row_stride,
                         void *stream) {
  const int feat = SWIGLU ? kFfnFeat : 2 * kFfnFeat;
  if (!x || !w || !out) return fail(SMLM_EINVAL, "%s: null x, weight or out pointer", what);
  if (M < 0 || K < 1 || N < 1)
    return fail(SMLM_EINVAL, "%s: bad shape M=%lld K=%d N=%d", what, (long long)M, K, N);
  if (K % kFfnKc || N % feat)
    return fail(SMLM_EUNSUPPORTED, "%s: K=%d must be a multiple of %d and %s=%d of %d", what, K, kFfnKc,
                SWIGLU ? "hidden" : "N", N, feat);
  if (x_row_stride < K || w_row_stride < K || out_row_stride < N || x_row_stride % 8 || w_row_stride % 8 ||
      out_row_stride % 8 || ((uintptr_t)x | (uintptr_t)w | (uintptr_t)out) % 16 || (uintptr_t)bias % 2)
    return fail(SMLM_EINVAL, "%s: rows must be 16-byte aligned with strides >= their widths (x %lld, weight %lld, "
                "out %lld)", what, (long long)x_row_stride, (long long)w_row_stride, (long long)out_row_stride);
  if (M == 0) return SMLM_OK;
  const int64_t ntt = (M + kFfnTok - 1) / kFfnTok;
  const int64_t grid = (ntt + kXcds - 1) / kXcds * kXcds * (N / feat);
  if (grid > 0x7FFFFFFFLL) return fail(SMLM_EUNSUPPORTED, "%s: M=%lld too large", what, (long long)M);
  hipLaunchKernelGGL((prompt_linear_kernel<SWIGLU>), dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t *)x, x_row_stride, (const uint16_t *)w, w_row_stride, (const uint16_t *)bias, M,
                     K, N, (uint16_t *)out, out_row_stride);
  return launch_status(what);
}

}  // namespace
}  // namespace smlm

extern "C" int smlm_linear_swiglu(const void *x, int64_t x_row_stride, const void *w13, int64_t w_row_stride,
                                  int64_t M, int K, int hidden, void *out, int64_t out_row_stride, void *stream) {
  return smlm::launch_prompt_linear<true>("smlm_linear_swiglu", x, x_row_stride, w13, w_row_stride, nullptr, M, K,
                                          hidden, out, out_row_stride, stream);
}

extern "C" int smlm_prompt_linear(const void *x, int64_t x_row_stride, const void *w, int64_t w_row_stride,
                                  const void *bias, int64_t M, int K, int N, void *out, int64_t out_row_stride,
                                  void *stream) {
  return smlm::launch_prompt_linear<false>("smlm_prompt_linear", x, x_row_stride, w, w_row_stride, bias, M, K, N,
                                           out, out_row_stride, stream);
}
