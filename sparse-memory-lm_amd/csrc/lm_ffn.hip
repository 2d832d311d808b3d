// Prompt-pass FFN up-projection with the SwiGLU activation in its epilogue (smlm/model.py:110-118):
//   out[m, j] = bf16(bf16(silu(a)) * b),  a = bf16(x[m] . w13[j]),  b = bf16(x[m] . w13[hidden + j])
// for the bf16 (M, K) activations x and the (2 hidden, K) nn.Linear weight w13, on v_mfma_f32_16x16x32_bf16 with
// fp32 accumulation: the roundings of the w13 projection (bf16 output) followed by smlm_swiglu, in one launch that
// writes the (M, hidden) activation only (the unfused pair writes and re-reads the (M, 2 hidden) projection).
//
// Workgroup = 4 wavefronts, a tile of 128 tokens x 64 output features: the 64 weight rows of a and the 64 of b,
// so each lane's a and b accumulators hold the same (token, feature) pairs.  Wavefront w: tokens 64 (w & 1) ..
// +63, features 32 (w >> 1) .. +31 (4 MFMA weight tiles: a lo / hi, b lo / hi x 4 token tiles).  K is staged in
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
constexpr int kFfnOutRow = kFfnFeat + 8;  // LDS row stride of the output tile (bf16)
constexpr int kFfnPieces = kFfnTok * kFfnKc / 8 / 256;  // 16-byte pieces per thread per operand per chunk (8)
constexpr int kXcds = 8;

__global__ void __launch_bounds__(256)
    ffn_swiglu_kernel(const uint16_t *__restrict__ x, int64_t x_stride, const uint16_t *__restrict__ w,
                      int64_t w_stride, int64_t M, int K, int hidden, uint16_t *__restrict__ out,
                      int64_t out_stride) {
  __shared__ __align__(16) uint16_t sW[2 * kFfnFeat * kFfnRow];  // weight rows: a features, then b features
  __shared__ __align__(16) uint16_t sX[kFfnTok * kFfnRow];       // token rows; later the output tile

  // tile: the feature blocks of token tile tt share an XCD
  const int nfb = hidden / kFfnFeat;
  const int64_t ntt = (M + kFfnTok - 1) / kFfnTok;
  const int64_t id = blockIdx.x, xcd = id % kXcds, local = id / kXcds;
  const int64_t tt = xcd + kXcds * (local / nfb);
  const int fb = (int)(local % nfb);
  if (tt >= ntt) return;  // workgroup-uniform, before any barrier
  const int64_t t0 = tt * kFfnTok;
  const int f0 = fb * kFfnFeat;

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
    const int64_t wrow = row < kFfnFeat ? f0 + row : (int64_t)hidden + f0 + (row - kFfnFeat);                 \
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
#define SMLM_FFN_WROW(i) (((i) >> 1) * kFfnFeat + fh * 32 + ((i) & 1) * 16)

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

  // epilogue: a, b rounded to bf16 as the projection's output, bf16(silu(a)) as smlm_swiglu, then bf16(s * b);
  // into the output tile in LDS (over the token rows, no longer read), then whole 128-byte row pieces to memory
  uint16_t *sO = sX;
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
      *(uint2 *)&sO[tok * kFfnOutRow + feat] = uint2{o[0], o[1]};
    }
  __syncthreads();
#pragma unroll
  for (int u = 0; u < kFfnTok * kFfnFeat / 8 / 256; ++u) {
    const int p = tid + 256 * u, row = p / 8, c = p % 8;
    if (t0 + row < M)
      *(uint4 *)(out + (t0 + row) * out_stride + f0 + c * 8) = *(const uint4 *)&sO[row * kFfnOutRow + c * 8];
  }
}

}  // namespace
}  // namespace smlm

extern "C" int smlm_linear_swiglu(const void *x, int64_t x_row_stride, const void *w13, int64_t w_row_stride,
                                  int64_t M, int K, int hidden, void *out, int64_t out_row_stride, void *stream) {
  using namespace smlm;
  if (!x || !w13 || !out) return fail(SMLM_EINVAL, "smlm_linear_swiglu: null x, w13 or out pointer");
  if (M < 0 || K < 1 || hidden < 1)
    return fail(SMLM_EINVAL, "smlm_linear_swiglu: bad shape M=%lld K=%d hidden=%d", (long long)M, K, hidden);
  if (K % kFfnKc || hidden % kFfnFeat)
    return fail(SMLM_EUNSUPPORTED, "smlm_linear_swiglu: K=%d must be a multiple of %d and hidden=%d of %d", K,
                kFfnKc, hidden, kFfnFeat);
  if (x_row_stride < K || w_row_stride < K || out_row_stride < hidden || x_row_stride % 8 || w_row_stride % 8 ||
      out_row_stride % 8 || ((uintptr_t)x | (uintptr_t)w13 | (uintptr_t)out) % 16)
    return fail(SMLM_EINVAL, "smlm_linear_swiglu: rows must be 16-byte aligned with strides >= their widths "
                "(x %lld, w13 %lld, out %lld)", (long long)x_row_stride, (long long)w_row_stride,
                (long long)out_row_stride);
  if (M == 0) return SMLM_OK;
  const int64_t ntt = (M + kFfnTok - 1) / kFfnTok;
  const int64_t grid = (ntt + kXcds - 1) / kXcds * kXcds * (hidden / kFfnFeat);
  if (grid > 0x7FFFFFFFLL) return fail(SMLM_EUNSUPPORTED, "smlm_linear_swiglu: M=%lld too large", (long long)M);
  hipLaunchKernelGGL(ffn_swiglu_kernel, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t *)x, x_row_stride, (const uint16_t *)w13, w_row_stride, M, K, hidden,
                     (uint16_t *)out, out_row_stride);
  return launch_status("smlm_linear_swiglu");
}
