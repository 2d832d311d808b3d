// Device helpers of the weighted value bag (kernel 4), shared by the bag kernels (pkm_bag.hip) and the fused
// decode selection + bag kernel (pkm_select.hip): table row formats, fp32 accumulation of 16-byte chunks,
// lookup staging and the output epilogue (swilu, bf16 rounding) of smlm/kernels.py:179-194, 304-361.
#pragma once

#include "pkm_common.h"

namespace smlm {
namespace bag {

enum TableKind { kF32 = SMLM_F32, kBF16 = SMLM_BF16, kI8 = SMLM_I8, kQ4 = SMLM_Q4 };

constexpr int kStage = 256;   // lookups staged in LDS per pass
constexpr int kUnroll = 8;    // independent 16-byte row loads in flight per thread

template <int TK>
constexpr int vals_per_chunk() {
  return TK == kF32 ? 4 : TK == kBF16 ? 8 : TK == kI8 ? 16 : 32;
}

// output column of value e of chunk c (q4: values 0..15 are the low nibbles = columns c*16+e, values 16..31
// the high nibbles = columns D/2 + c*16 + e)
template <int TK>
__device__ __forceinline__ int chunk_col(int c, int e, int D) {
  if constexpr (TK == kQ4) return e < 16 ? c * 16 + e : (D >> 1) + c * 16 + (e - 16);
  else return c * vals_per_chunk<TK>() + e;
}

template <int TK>
__device__ __forceinline__ void accumulate(float *acc, const uint4 v, const float wt) {
  const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    if constexpr (TK == kF32) {
      acc[e] = fmaf(wt, __uint_as_float(u[e]), acc[e]);
    } else if constexpr (TK == kBF16) {
      acc[2 * e] = fmaf(wt, __uint_as_float(u[e] << 16), acc[2 * e]);
      acc[2 * e + 1] = fmaf(wt, __uint_as_float(u[e] & 0xFFFF0000u), acc[2 * e + 1]);
    } else if constexpr (TK == kI8) {
#pragma unroll
      for (int b = 0; b < 4; ++b)
        acc[4 * e + b] = fmaf(wt, (float)(int8_t)(u[e] >> (8 * b)), acc[4 * e + b]);
    } else {
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int byte = (int)((u[e] >> (8 * b)) & 0xFFu);
        acc[4 * e + b] = fmaf(wt, (float)((byte & 15) - 8), acc[4 * e + b]);
        acc[16 + 4 * e + b] = fmaf(wt, (float)((byte >> 4) - 8), acc[16 + 4 * e + b]);
      }
    }
  }
}

// value of column `col` of a row (generic kernel)
template <int TK>
__device__ __forceinline__ float row_value(const uint8_t *row, int col, int D) {
  if constexpr (TK == kF32) return ((const float *)row)[col];
  else if constexpr (TK == kBF16) return bf16_bits_to_f32(((const uint16_t *)row)[col]);
  else if constexpr (TK == kI8) return (float)((const int8_t *)row)[col];
  else {
    const int half = D >> 1;
    const int byte = row[col < half ? col : col - half];
    return (float)((col < half ? (byte & 15) : (byte >> 4)) - 8);
  }
}

// Stage lookups [k0, k0 + kc) of token n: byte offset of the row and weight (times the row scale).  An index
// outside [0, rows) contributes nothing and marks the token bad.
template <int TK, bool IDX64>
__device__ __forceinline__ void stage_lookups(const void *__restrict__ idx, const float *__restrict__ w,
                                              const uint16_t *__restrict__ scales, int64_t base, int kc,
                                              int64_t rows, int64_t row_bytes, int64_t *s_off, float *s_w,
                                              int *s_bad) {
  for (int j = threadIdx.x; j < kc; j += blockDim.x) {
    int64_t r = IDX64 ? ((const int64_t *)idx)[base + j] : (int64_t)((const int32_t *)idx)[base + j];
    float wt = w[base + j];
    if (r < 0 || r >= rows) {
      *s_bad = 1;
      r = 0;
      wt = 0.f;
    }
    if constexpr (TK == kI8 || TK == kQ4) wt *= f16_bits_to_f32(scales[r]);
    s_off[j] = r * row_bytes;
    s_w[j] = wt;
  }
}

// out[o] = a (NaN for a bad token), times bf16(silu(pre)) when has_pre (pre_bits = the bf16 bits of pre[o])
__device__ __forceinline__ void store_out_bits(void *out, int64_t o, float a, bool bad, bool has_pre,
                                               uint16_t pre_bits, bool out_bf16) {
  if (bad) a = __builtin_nanf("");
  if (has_pre) {
    const float p = bf16_bits_to_f32(pre_bits);
    a *= round_bf16(p / (1.0f + expf(-p)));  // bf16(silu(pre)), as smlm/kernels.py:304-307
  }
  if (out_bf16) ((uint16_t *)out)[o] = (uint16_t)bf16_bits_rtne(a);
  else ((float *)out)[o] = a;
}

__device__ __forceinline__ void store_out(void *out, int64_t o, float a, bool bad, const uint16_t *pre,
                                          bool out_bf16) {
  store_out_bits(out, o, a, bad, pre != nullptr, pre ? pre[o] : (uint16_t)0, out_bf16);
}

// Rows of a token's staged lookups [0, kc) accumulated by row slot `slot` of a layout of rpr row slots x cpr chunk
// columns: thread (slot, c) adds w_j * chunk c of row j for j = slot, slot + rpr, ... in that order (UNROLL loads in
// flight; the order of the additions does not depend on UNROLL).  The rounds are unpredicated: selecting a loaded
// value under a lane condition made the compiler wait for each load before issuing the next (the config-4 Zipf
// gather 386 -> 470 us, the decode step +3 us).
template <int TK, int UNROLL = kUnroll>
__device__ __forceinline__ void accumulate_rows(const uint8_t *__restrict__ colbase, int slot, int rpr, int kc,
                                                const int64_t *s_off, const float *s_w, float *acc) {
  int j = slot;
  for (; j + (UNROLL - 1) * rpr < kc; j += UNROLL * rpr) {
    uint4 v[UNROLL];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) v[u] = *(const uint4 *)(colbase + s_off[j + u * rpr]);
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) accumulate<TK>(acc, v[u], s_w[j + u * rpr]);
  }
  for (; j < kc; j += rpr) accumulate<TK>(acc, *(const uint4 *)(colbase + s_off[j]), s_w[j]);
}

// Threads of the canonical row-slot layout for rows of cpr 16-byte chunks: as many whole rows (slots) as fit in
// kBagThreads threads for rows of up to 32 chunks (int8 rows of 384 values, 24 chunks: 8 slots; q4, 12: 16), in
// kBagThreadsWide for wider rows (bf16, 48: 8 slots; fp32, 96: 4), one slot at least.  The slot count fixes the
// order of the fp32 additions (each slot sums its rows in order, then the slots are added in slot order), so every
// kernel that must agree bit for bit uses this layout; a workgroup with fewer threads runs several slots per
// thread (select_bag_kernel).  Measured (MI355X): 16 int8 slots in 384 threads took the config-4 gather 652 ->
// 732 us (uniform) and 389 -> 588 us (Zipf); 8 bf16 slots instead of 4 took the decode step 177.1 -> 176.5 us
// (batch 64) and 124.3 -> 123.5 us (batch 1) with the config-2 bf16 bag unchanged (279-280 us).
constexpr int kBagThreads = 192;
constexpr int kBagThreadsWide = 384;
constexpr int kBagMaxChunks = 256;     // rows of more 16-byte chunks take the generic kernel
constexpr int imax(int a, int b) { return a > b ? a : b; }
// the most threads bag_threads returns for rows of at most kBagMaxChunks chunks (a slot budget, or one slot of
// up to kBagMaxChunks threads): the launch bound of the kernels that run this layout in one workgroup (launching
// more threads than a kernel's bound fails)
constexpr int kBagMaxThreads = imax(kBagMaxChunks, imax(kBagThreads, kBagThreadsWide));

__host__ __device__ constexpr int bag_slots(int cpr) {
  return cpr >= (cpr <= 32 ? kBagThreads : kBagThreadsWide) ? 1 : (cpr <= 32 ? kBagThreads : kBagThreadsWide) / cpr;
}
__host__ __device__ constexpr int bag_threads(int cpr) { return bag_slots(cpr) * cpr; }

}  // namespace bag
}  // namespace smlm
