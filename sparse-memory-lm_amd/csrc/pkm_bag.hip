// Weighted value bag (kernel 4): out[n, :] = sum_j w[n, j] * row(idx[n, j]) with fp32 accumulation, for fp32,
// bf16, int8 (+fp16 row scale) and packed 4-bit (+fp16 row scale) tables; optional swilu epilogue and bf16
// output.  Replaces bag_forward / bag_infer of smlm/kernels.py:179-194, 229-237, 313-378.
//
// The gather is HBM-bound: every lookup reads one whole table row (768 B for a 384-wide bf16 row).  One
// workgroup owns one token.  A row is cut into 16-byte chunks (cpr chunks per row) and the workgroup's threads
// are laid out as rpr row slots x cpr chunk columns, so one "round" of the workgroup reads rpr whole rows with
// coalesced 16-byte loads and every lane is busy (384-wide rows: 192 threads = 4 bf16 / 8 int8 / 2 fp32 /
// 16 q4 rows per round).  Each thread keeps the fp32 partial sums of its chunk's columns over the rows of its
// slot and issues kUnroll independent row loads at a time; the rpr partial sums per column are added through
// LDS at the end, followed by the epilogue.  Lookups (row offsets, weights premultiplied by the row scale) are
// staged in LDS first, so each row load depends on one LDS read only.
#include "pkm_common.h"

namespace smlm {
namespace {

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

__device__ __forceinline__ void store_out(void *out, int64_t o, float a, bool bad, const uint16_t *pre,
                                          bool out_bf16) {
  if (bad) a = __builtin_nanf("");
  if (pre) {
    const float p = bf16_bits_to_f32(pre[o]);
    a *= round_bf16(p / (1.0f + expf(-p)));  // bf16(silu(pre)), as smlm/kernels.py:304-307
  }
  if (out_bf16) ((uint16_t *)out)[o] = (uint16_t)bf16_bits_rtne(a);
  else ((float *)out)[o] = a;
}

template <int TK, bool IDX64>
__global__ void __launch_bounds__(256) bag_rows_kernel(const void *__restrict__ idx, const float *__restrict__ w,
                                                       const uint8_t *__restrict__ table,
                                                       const uint16_t *__restrict__ scales,
                                                       const uint16_t *__restrict__ pre, void *__restrict__ out,
                                                       int K, int D, int64_t rows, int row_bytes, int cpr,
                                                       int out_bf16) {
  constexpr int VPC = vals_per_chunk<TK>();
  extern __shared__ __align__(16) unsigned char smem[];
  int64_t *s_off = (int64_t *)smem;           // [kStage]
  float *s_w = (float *)(s_off + kStage);     // [kStage]
  float *s_red = s_w + kStage;                // [rpr][D]
  __shared__ int s_bad;

  const int tid = threadIdx.x;
  const int rpr = blockDim.x / cpr;
  const int c = tid % cpr;
  const int slot = tid / cpr;
  const int64_t n = blockIdx.x;
  const int64_t lbase = n * (int64_t)K;
  const uint8_t *colbase = table + (int64_t)c * 16;
  if (tid == 0) s_bad = 0;

  float acc[VPC];
#pragma unroll
  for (int e = 0; e < VPC; ++e) acc[e] = 0.f;

  for (int k0 = 0; k0 < K; k0 += kStage) {
    const int kc = min(kStage, K - k0);
    __syncthreads();  // previous pass has finished reading s_off / s_w
    stage_lookups<TK, IDX64>(idx, w, scales, lbase + k0, kc, rows, row_bytes, s_off, s_w, &s_bad);
    __syncthreads();
    int j = slot;
    for (; j + (kUnroll - 1) * rpr < kc; j += kUnroll * rpr) {
      uint4 v[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) v[u] = *(const uint4 *)(colbase + s_off[j + u * rpr]);
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) accumulate<TK>(acc, v[u], s_w[j + u * rpr]);
    }
    for (; j < kc; j += rpr) accumulate<TK>(acc, *(const uint4 *)(colbase + s_off[j]), s_w[j]);
  }

#pragma unroll
  for (int e = 0; e < VPC; ++e) s_red[slot * D + chunk_col<TK>(c, e, D)] = acc[e];
  __syncthreads();
  const bool bad = s_bad != 0;
  for (int col = tid; col < D; col += blockDim.x) {
    float a = 0.f;
    for (int r = 0; r < rpr; ++r) a += s_red[r * D + col];
    store_out(out, n * D + col, a, bad, pre, out_bf16);
  }
}

// Any row width: one thread per output column (rows whose byte width is not a multiple of 16, or very wide).
template <int TK, bool IDX64>
__global__ void __launch_bounds__(256) bag_generic_kernel(const void *__restrict__ idx,
                                                          const float *__restrict__ w,
                                                          const uint8_t *__restrict__ table,
                                                          const uint16_t *__restrict__ scales,
                                                          const uint16_t *__restrict__ pre, void *__restrict__ out,
                                                          int K, int D, int64_t rows, int row_bytes, int out_bf16) {
  __shared__ int64_t s_off[kStage];
  __shared__ float s_w[kStage];
  __shared__ int s_bad;
  const int64_t n = blockIdx.x;
  const int col = blockIdx.y * blockDim.x + threadIdx.x;
  const int64_t lbase = n * (int64_t)K;
  if (threadIdx.x == 0) s_bad = 0;
  float a = 0.f;
  for (int k0 = 0; k0 < K; k0 += kStage) {
    const int kc = min(kStage, K - k0);
    __syncthreads();
    stage_lookups<TK, IDX64>(idx, w, scales, lbase + k0, kc, rows, row_bytes, s_off, s_w, &s_bad);
    __syncthreads();
    if (col < D)
      for (int j = 0; j < kc; ++j) a = fmaf(s_w[j], row_value<TK>(table + s_off[j], col, D), a);
  }
  __syncthreads();
  if (col < D) store_out(out, n * D + col, a, s_bad != 0, pre, out_bf16);
}

template <int TK, bool IDX64>
int launch_bag(const void *idx, const float *w, int64_t N, int K, const void *table, int64_t rows, int D,
               const uint16_t *scales, const uint16_t *pre, void *out, int out_bf16, hipStream_t stream) {
  const int64_t row_bytes64 = TK == kF32 ? 4LL * D : TK == kBF16 ? 2LL * D : TK == kI8 ? (int64_t)D : D / 2;
  const int row_bytes = (int)row_bytes64;
  const bool aligned = ((uintptr_t)table % 16) == 0;
  const int cpr = row_bytes / 16;
  if (aligned && row_bytes % 16 == 0 && cpr >= 1 && cpr <= 256) {
    // threads = lcm(cpr, 64) (whole wavefronts, every lane busy), at least 128; else as many row slots as fit
    int g = cpr, b = kWave;
    while (b) { const int t = g % b; g = b; b = t; }
    int nthr = cpr / g * kWave;
    if (nthr > 256) nthr = cpr * (256 / cpr);
    while (nthr < 128) nthr *= 2;
    const int rpr = nthr / cpr;
    const size_t shmem = kStage * (sizeof(int64_t) + sizeof(float)) + (size_t)rpr * D * sizeof(float);
    hipLaunchKernelGGL((bag_rows_kernel<TK, IDX64>), dim3((unsigned)N), dim3(nthr), shmem, stream, idx, w,
                       (const uint8_t *)table, scales, pre, out, K, D, rows, row_bytes, cpr, out_bf16);
  } else {
    const int nthr = 256;
    hipLaunchKernelGGL((bag_generic_kernel<TK, IDX64>), dim3((unsigned)N, (unsigned)((D + nthr - 1) / nthr)),
                       dim3(nthr), 0, stream, idx, w, (const uint8_t *)table, scales, pre, out, K, D, rows,
                       row_bytes, out_bf16);
  }
  return launch_status("smlm_pkm_bag");
}

template <int TK>
int launch_bag_idx(int idx64, const void *idx, const float *w, int64_t N, int K, const void *table, int64_t rows,
                   int D, const uint16_t *scales, const uint16_t *pre, void *out, int out_bf16,
                   hipStream_t stream) {
  return idx64 ? launch_bag<TK, true>(idx, w, N, K, table, rows, D, scales, pre, out, out_bf16, stream)
               : launch_bag<TK, false>(idx, w, N, K, table, rows, D, scales, pre, out, out_bf16, stream);
}

}  // namespace
}  // namespace smlm

extern "C" int smlm_pkm_bag(const void *idx, int idx_dtype, const float *w, int64_t N, int K, const void *table,
                            int table_dtype, int64_t rows, int D, const uint16_t *scales, const uint16_t *pre,
                            void *out, int out_dtype, void *stream) {
  using namespace smlm;
  if (!idx || !w || !table || !out) return fail(SMLM_EINVAL, "smlm_pkm_bag: null idx, w, table or out pointer");
  if (N < 0 || N > 0x7FFFFFFFLL) return fail(SMLM_EINVAL, "smlm_pkm_bag: N=%lld out of range", (long long)N);
  if (K < 1) return fail(SMLM_EINVAL, "smlm_pkm_bag: K=%d must be >= 1", K);
  if (D < 1) return fail(SMLM_EINVAL, "smlm_pkm_bag: D=%d must be >= 1", D);
  if (rows < 1) return fail(SMLM_EINVAL, "smlm_pkm_bag: rows=%lld must be >= 1", (long long)rows);
  if (idx_dtype != SMLM_I64 && idx_dtype != SMLM_I32)
    return fail(SMLM_EINVAL, "smlm_pkm_bag: idx_dtype must be SMLM_I64 or SMLM_I32, got %d", idx_dtype);
  if (out_dtype != SMLM_F32 && out_dtype != SMLM_BF16)
    return fail(SMLM_EINVAL, "smlm_pkm_bag: out_dtype must be SMLM_F32 or SMLM_BF16, got %d", out_dtype);
  const bool quant = table_dtype == SMLM_I8 || table_dtype == SMLM_Q4;
  if (table_dtype != SMLM_F32 && table_dtype != SMLM_BF16 && !quant)
    return fail(SMLM_EINVAL, "smlm_pkm_bag: table_dtype %d is not f32, bf16, i8 or q4", table_dtype);
  if (quant != (scales != nullptr))
    return fail(SMLM_EINVAL, "smlm_pkm_bag: row scales are required for i8/q4 tables and only for them");
  if (table_dtype == SMLM_Q4 && D % 2)
    return fail(SMLM_EINVAL, "smlm_pkm_bag: q4 tables need an even D, got %d", D);
  if (N == 0) return SMLM_OK;
  const int idx64 = idx_dtype == SMLM_I64;
  const int ob = out_dtype == SMLM_BF16;
  hipStream_t s = (hipStream_t)stream;
  switch (table_dtype) {
    case SMLM_F32: return launch_bag_idx<kF32>(idx64, idx, w, N, K, table, rows, D, scales, pre, out, ob, s);
    case SMLM_BF16: return launch_bag_idx<kBF16>(idx64, idx, w, N, K, table, rows, D, scales, pre, out, ob, s);
    case SMLM_I8: return launch_bag_idx<kI8>(idx64, idx, w, N, K, table, rows, D, scales, pre, out, ob, s);
    default: return launch_bag_idx<kQ4>(idx64, idx, w, N, K, table, rows, D, scales, pre, out, ob, s);
  }
}
