// Prompt-pass projections on the matrix cores (v_mfma_f32_16x16x32_bf16, fp32 accumulation), bf16 activations x
// (M, K) and nn.Linear weights:
//   smlm_linear_swiglu: the FFN up-projection with the SwiGLU activation in its epilogue (smlm/model.py:110-118),
//     out[m, j] = bf16(bf16(silu(a)) * b), a = bf16(x[m] . w13[j]), b = bf16(x[m] . w13[hidden + j]): the roundings
//     of the w13 projection (bf16 output) followed by smlm_swiglu, in one launch that writes the (M, hidden)
//     activation only (the unfused pair writes and re-reads the (M, 2 hidden) projection);
//   smlm_prompt_linear: out = bf16(x W^T + bias) for the other projections of a prompt pass (wqkv, wo, w2, the
//     memory layer's swilu_proj and value_proj), where the library GEMMs' large tiles leave CUs idle, and with an
//     fp32 per-column scale / shift on the bf16 result the memory query with its eval BatchNorm (smlm/pkm.py:188-191).
//
// Workgroup = 4 wavefronts, a tile of 128 tokens x 128 weight rows.  SwiGLU: the 64 weight rows of a and the 64
// of b, so each lane's a and b accumulators hold the same (token, feature) pairs; wavefront w: tokens 64 (w & 1)
// .. +63, features 32 (w >> 1) .. +31 (4 MFMA weight tiles: a lo / hi, b lo / hi x 4 token tiles).  Plain: 128
// output features, wavefront w: tokens 64 (w & 1) .., features 64 (w >> 1) .. +63.
//
// K streams through LDS in chunks of 64 (two stages): each chunk is loaded straight from global memory into LDS
// (global_load_lds_dwordx4, no registers in between), the next chunk's loads run during this chunk's products, and
// one barrier per chunk both publishes the chunk and frees the stage it reloads.  A stage holds the 128 weight rows
// and the 128 token rows, 128 bytes each, piece c of row R at position c ^ ((R / 2) % 8), so that the 16 rows of a
// fragment read fall on distinct banks.  1-D grid, XCD-aware: the workgroups of one XCD (workgroup id % 8) walk
// its token tiles fastest, so the ~64 it runs at once share a few token tiles and weight blocks through its L2.
//
// MFMA operand mapping (16x16x32, r = lane % 16, g = lane / 16): A = 16 weight rows x 32 k (lane: row r, k group
// g), B = 32 k x 16 tokens (lane: token r, k group g), D: lane holds features 4g..4g+3 of token r.
#include "pkm_common.h"

namespace smlm {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) unsigned char lds_u8;

constexpr int kFfnTok = 128;                          // tokens per workgroup
constexpr int kFfnRows = 128;                         // weight rows per workgroup
constexpr int kFfnFeat = 64;                          // SwiGLU: output features per workgroup (+ their 64 b rows)
constexpr int kFfnKc = 64;                            // K chunk per stage
constexpr int kRowBytes = kFfnKc * 2;                 // 128: a chunk row
constexpr int kStage = (kFfnRows + kFfnTok) * kRowBytes;   // 32 KB: weight rows, then token rows
constexpr int kLoads = kStage / 4096;                 // direct loads per thread per chunk (1 KB per wavefront each)
constexpr int kWeightLoads = kFfnRows * kRowBytes / 4096;
constexpr int kXcds = 8;

// 16 bytes per lane from global memory straight into LDS: from sbase + voff (a wave-uniform 64-bit base and the
// lane's 32-bit byte offset) to LDS lds_base + 16 * lane (wave-uniform).  Inline assembly, so that the compiler adds
// no vmcnt(0) wait for the LDS it writes before every LDS read (it cannot tell the two stages apart): the kernel
// waits for these loads itself (wait_loads) before the barrier that publishes a chunk.  M0 is set right before the
// load; nothing else in the kernel uses M0.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void load_lds16(const void *sbase, uint32_t voff, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "s"(lds_base) : "m0");
}
#pragma clang diagnostic pop

// s_waitcnt vmcnt(N): at most N vector memory operations of this wavefront outstanding.  Loads complete in order,
// so with N = the loads issued after chunk ch's, chunk ch has landed.
template <int N>
__device__ __forceinline__ void wait_loads() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}

// SWIGLU: the stage's 128 weight rows are the a rows f0 .. f0 + 63 and the b rows hidden + f0 .. (64 output
// features); otherwise (plain projection, bf16 out) the rows f0 .. f0 + 127 (128 output features, N = hidden).
template <bool SWIGLU>
__global__ void __launch_bounds__(256)
    prompt_linear_kernel(const uint16_t *__restrict__ x, int64_t x_stride, const uint16_t *__restrict__ w,
                         int64_t w_stride, const uint16_t *__restrict__ bias, const float *__restrict__ scale,
                         const float *__restrict__ shift, int64_t M, int K, int hidden, uint16_t *__restrict__ out,
                         int64_t out_stride) {
  constexpr int FEAT = SWIGLU ? kFfnFeat : kFfnRows;   // output features per workgroup
  __shared__ __align__(16) unsigned char stages[2 * kStage];

  // tile: an XCD owns the token tiles xcd, xcd + 8, ..; its workgroups take them token tile fastest
  const int nfb = hidden / FEAT;
  const int64_t ntt = (M + kFfnTok - 1) / kFfnTok, t8 = (ntt + kXcds - 1) / kXcds;
  const int64_t id = blockIdx.x, xcd = id % kXcds, local = id / kXcds;
  const int64_t tt = xcd + kXcds * (local % t8);
  const int fb = (int)(local / t8);
  if (tt >= ntt || fb >= nfb) return;  // workgroup-uniform, before any barrier
  const int64_t t0 = tt * kFfnTok;
  const int f0 = fb * FEAT;

  const int tid = threadIdx.x, wave = tid / kWave, lane = lane_id();
  const int r = lane & 15, g = lane >> 4;
  const int th = wave & 1, fh = wave >> 1;

  // load u of wavefront `wave` fills stage rows 32 u + 8 wave .. + 7 (lane: row + lane / 8, position lane % 8,
  // so it loads piece (lane % 8) ^ ((row / 2) % 8)); loads 0-3 are weight rows, 4-7 token rows (rows past M read
  // row M - 1, whose results are not stored).  Rows 32 apart share the swizzle, so each lane keeps one byte offset
  // per operand row (fixed over the chunks) and the row steps and chunk advance go into the wave-uniform base.
  const uint32_t wv = __builtin_amdgcn_readfirstlane(wave);
  const int wl = wave * 8 + lane / 8;
  const int cpos = (lane % 8) ^ ((wl >> 1) & 7);
  const uint32_t woff = (uint32_t)(((int64_t)wl * w_stride + cpos * 8) * 2);
  uint32_t xoff[kLoads - kWeightLoads];
#pragma unroll
  for (int u = 0; u < kLoads - kWeightLoads; ++u)
    xoff[u] = (uint32_t)(((min(t0 + 32 * u + wl, M - 1) - t0) * x_stride + cpos * 8) * 2);
  const uint16_t *xt = x + t0 * x_stride;
  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_u8 *)stages + wv * 1024;
  auto issue = [&](int ch, uint32_t stage_off) {
    const int k0 = ch * kFfnKc;
#pragma unroll
    for (int u = 0; u < kLoads; ++u) {
      if (u < kWeightLoads) {
        const int64_t row0 = !SWIGLU || 32 * u < kFfnFeat ? (int64_t)f0 + 32 * u : (int64_t)hidden + f0 + 32 * u - kFfnFeat;
        load_lds16(w + row0 * w_stride + k0, woff, lds0 + stage_off + u * 4096);
      } else {
        load_lds16(xt + k0, xoff[u - kWeightLoads], lds0 + stage_off + u * 4096);
      }
    }
  };

  floatx4 acc[4][4];  // [weight tile: a lo, a hi, b lo, b hi][token tile]
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
// the stage row of weight tile i: SWIGLU: tiles a lo, a hi, b lo, b hi of features fh * 32 .. +31; otherwise 4
// tiles of features fh * 64 .. +63
#define SMLM_FFN_WROW(i) (SWIGLU ? ((i) >> 1) * kFfnFeat + fh * 32 + ((i) & 1) * 16 : fh * 64 + (i) * 16)
  auto compute = [&](const unsigned char *st) {
#pragma unroll
    for (int s = 0; s < kFfnKc / 32; ++s) {
      const int c = s * 4 + g;
      bf16x8 a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int R = SMLM_FFN_WROW(i) + r;
        a[i] = *(const bf16x8 *)(st + R * kRowBytes + (c ^ ((R >> 1) & 7)) * 16);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int R = kFfnRows + th * 64 + j * 16 + r;
        b[j] = *(const bf16x8 *)(st + R * kRowBytes + (c ^ ((R >> 1) & 7)) * 16);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
  };
#undef SMLM_FFN_WROW

  // chunk ch lives in stage ch % 2; the loop is unrolled by two so that each stage's offset is a constant
  const int nch = K / kFfnKc;
  auto step = [&](int ch, uint32_t this_off, uint32_t other_off) {
    wait_loads<0>();   // chunk ch landed (the only loads in flight)
    __syncthreads();   // chunk ch visible to every wavefront; every wavefront is done with chunk ch - 1
    if (ch + 1 < nch) issue(ch + 1, other_off);   // into the stage of chunk ch - 1, in flight during these products
    compute(stages + this_off);
  };
  issue(0, 0);
  int ch = 0;
  for (; ch + 1 < nch; ch += 2) {
    step(ch, 0, kStage);
    step(ch + 1, kStage, 0);
  }
  if (ch < nch) step(ch, 0, kStage);
  __syncthreads();     // every wavefront is done with the stages

  // epilogue through LDS (the stages), stored as whole 128-byte row pieces.  SWIGLU: a, b rounded to bf16 as the
  // projection's output, bf16(silu(a)) as smlm_swiglu, then bf16(s * b), into the workgroup's 128 x 64 tile;
  // otherwise the projection plus its bias (fp32) rounded to bf16 (with scale / shift: that bf16 value times scale
  // plus shift, in fp32, rounded again), each wavefront its own 64 x 64 tile.  The roundings use v_cvt_pk_bf16_f32
  // (round to nearest even: the integer rounding's bits for finite values).
  if constexpr (SWIGLU) {
    constexpr int OROW = kFfnFeat + 8;
    uint16_t *sO = (uint16_t *)stages;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint32_t o[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          float h[2];
#pragma unroll
          for (int q = 0; q < 2; ++q) {
            const float av = round_bf16_hw(acc[i][j][2 * e + q]);
            const float bv = round_bf16_hw(acc[2 + i][j][2 * e + q]);
            const float sv = round_bf16_hw(av / (1.0f + expf(-av)));
            h[q] = sv * bv;
          }
          o[e] = pack_bf16x2(h[0], h[1]);
        }
        const int tok = th * 64 + j * 16 + r, feat = fh * 32 + i * 16 + 4 * g;
        *(uint2 *)&sO[tok * OROW + feat] = uint2{o[0], o[1]};
      }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < kFfnTok * 8 / 256; ++u) {
      const int p = tid + 256 * u, row = p / 8, c = p % 8;
      if (t0 + row < M)
        *(uint4 *)(out + (t0 + row) * out_stride + f0 + c * 8) = *(const uint4 *)&sO[row * OROW + c * 8];
    }
  } else {
    constexpr int OROW = 64 + 8;
    uint16_t *sO = (uint16_t *)stages + wave * 64 * OROW;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int col = f0 + fh * 64 + i * 16 + 4 * g;
      float bv[4] = {0.f, 0.f, 0.f, 0.f};
      if (bias) {
#pragma unroll
        for (int e = 0; e < 4; ++e) bv[e] = bf16_bits_to_f32(bias[col + e]);
      }
      float4 sc = {1.f, 1.f, 1.f, 1.f}, sh = {0.f, 0.f, 0.f, 0.f};
      if (scale) {
        sc = *(const float4 *)(scale + col);
        sh = *(const float4 *)(shift + col);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = acc[i][j][e] + bv[e];
        if (scale) {   // the eval BatchNorm on the bf16 projection: bf16(bf16(v) * scale + shift)
          v[0] = fmaf(round_bf16_hw(v[0]), sc.x, sh.x);
          v[1] = fmaf(round_bf16_hw(v[1]), sc.y, sh.y);
          v[2] = fmaf(round_bf16_hw(v[2]), sc.z, sh.z);
          v[3] = fmaf(round_bf16_hw(v[3]), sc.w, sh.w);
        }
        *(uint2 *)&sO[(j * 16 + r) * OROW + i * 16 + 4 * g] = uint2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
      }
    }
    // each wavefront reads back only what it wrote: no barrier
#pragma unroll
    for (int u = 0; u < 64 * 8 / 64; ++u) {
      const int p = lane + 64 * u, row = p / 8, c = p % 8;
      const int64_t t = t0 + th * 64 + row;
      if (t < M) *(uint4 *)(out + t * out_stride + f0 + fh * 64 + c * 8) = *(const uint4 *)&sO[row * OROW + c * 8];
    }
  }
}

}  // namespace
}  // namespace smlm

namespace smlm {
namespace {

// shared checks and launch: N = the kernel's `hidden` (SWIGLU: the activation's width; otherwise the output width)
template <bool SWIGLU>
int launch_prompt_linear(const char *what, const void *x, int64_t x_row_stride, const void *w, int64_t w_row_stride,
                         const void *bias, const float *scale, const float *shift, int64_t M, int K, int N, void *out,
                         int64_t out_row_stride, void *stream) {
  const int feat = SWIGLU ? kFfnFeat : kFfnRows;
  if (!x || !w || !out) return fail(SMLM_EINVAL, "%s: null x, weight or out pointer", what);
  if ((scale == nullptr) != (shift == nullptr) || ((uintptr_t)scale | (uintptr_t)shift) % 16)
    return fail(SMLM_EINVAL, "%s: scale and shift must both be given (16-byte aligned fp32) or both be null", what);
  if (M < 0 || K < 1 || N < 1)
    return fail(SMLM_EINVAL, "%s: bad shape M=%lld K=%d N=%d", what, (long long)M, K, N);
  if (K % kFfnKc || N % feat)
    return fail(SMLM_EUNSUPPORTED, "%s: K=%d must be a multiple of %d and %s=%d of %d", what, K, kFfnKc,
                SWIGLU ? "hidden" : "N", N, feat);
  // the lanes' 32-bit byte offsets into a 128-row tile: strides up to 2^24 elements
  if (x_row_stride > (1 << 24) || w_row_stride > (1 << 24))
    return fail(SMLM_EUNSUPPORTED, "%s: row strides above 2^24 elements (x %lld, weight %lld)", what,
                (long long)x_row_stride, (long long)w_row_stride);
  if (x_row_stride < K || w_row_stride < K || out_row_stride < N || x_row_stride % 8 || w_row_stride % 8 ||
      out_row_stride % 8 || ((uintptr_t)x | (uintptr_t)w | (uintptr_t)out) % 16 || (uintptr_t)bias % 2)
    return fail(SMLM_EINVAL, "%s: rows must be 16-byte aligned with strides >= their widths (x %lld, weight %lld, "
                "out %lld)", what, (long long)x_row_stride, (long long)w_row_stride, (long long)out_row_stride);
  if (M == 0) return SMLM_OK;
  const int64_t ntt = (M + kFfnTok - 1) / kFfnTok;
  const int64_t grid = (ntt + kXcds - 1) / kXcds * kXcds * (N / feat);
  if (grid > 0x7FFFFFFFLL) return fail(SMLM_EUNSUPPORTED, "%s: M=%lld too large", what, (long long)M);
  hipLaunchKernelGGL((prompt_linear_kernel<SWIGLU>), dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t *)x, x_row_stride, (const uint16_t *)w, w_row_stride, (const uint16_t *)bias, scale,
                     shift, M, K, N, (uint16_t *)out, out_row_stride);
  return launch_status(what);
}

}  // namespace
}  // namespace smlm

extern "C" int smlm_linear_swiglu(const void *x, int64_t x_row_stride, const void *w13, int64_t w_row_stride,
                                  int64_t M, int K, int hidden, void *out, int64_t out_row_stride, void *stream) {
  return smlm::launch_prompt_linear<true>("smlm_linear_swiglu", x, x_row_stride, w13, w_row_stride, nullptr, nullptr,
                                          nullptr, M, K, hidden, out, out_row_stride, stream);
}

extern "C" int smlm_prompt_linear(const void *x, int64_t x_row_stride, const void *w, int64_t w_row_stride,
                                  const void *bias, const float *scale, const float *shift, int64_t M, int K, int N,
                                  void *out, int64_t out_row_stride, void *stream) {
  return smlm::launch_prompt_linear<false>("smlm_prompt_linear", x, x_row_stride, w, w_row_stride, bias, scale, shift,
                                           M, K, N, out, out_row_stride, stream);
}
