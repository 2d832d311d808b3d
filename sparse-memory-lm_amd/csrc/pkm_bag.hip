// Weighted value bag (kernel 4): out[n, :] = sum_j w[n, j] * row(idx[n, j]) with fp32 accumulation, for fp32,
// bf16, int8 (+fp16 row scale) and packed 4-bit (+fp16 row scale) tables; optional swilu epilogue and bf16
// output.  Replaces bag_forward / bag_infer of smlm/kernels.py:179-194, 229-237, 313-378.
//
// The gather is HBM-bound: every lookup reads one whole table row (768 B for a 384-wide bf16 row).  One
// workgroup owns one token.  A row is cut into 16-byte chunks (cpr chunks per row) and the workgroup's threads
// are laid out as rpr row slots x cpr chunk columns (bag::bag_threads: 8 int8 / 16 q4 rows of 384 values in 192
// threads, 8 bf16 / 4 fp32 rows in 384), so each round reads rpr whole rows with coalesced 16-byte loads and every
// lane is busy.  Each thread keeps the fp32 partial sums of its chunk's columns over the rows of its slot and
// issues kUnroll independent row loads at a time; the rpr partial sums per column are added through LDS at the
// end, followed by the epilogue.  Lookups (row offsets, weights premultiplied by the row scale) are staged in LDS
// first, one per thread, so each row load depends on one LDS read only.  Loading each lookup's index, weight and
// scale in every lane of its slot instead of staging them measured 0.87 against 0.65 ms at config 4 (uniform):
// three redundant memory instructions per row load.
#include "pkm_bag_dev.h"

namespace smlm {
namespace {

using namespace bag;

template <int TK, bool IDX64>
__global__ void __launch_bounds__(kBagMaxThreads)
    bag_rows_kernel(const void *__restrict__ idx, const float *__restrict__ w, const uint8_t *__restrict__ table,
                    const uint16_t *__restrict__ scales, const uint16_t *__restrict__ pre, void *__restrict__ out,
                    int K, int D, int64_t rows, int row_bytes, int cpr, int out_bf16) {
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
    accumulate_rows<TK>(colbase, slot, rpr, kc, s_off, s_w, acc);
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
  if (aligned && row_bytes % 16 == 0 && cpr >= 1 && cpr <= kBagMaxChunks) {
    const int nthr = bag_threads(cpr);
    if (nthr > kBagMaxThreads)
      return fail(SMLM_EUNSUPPORTED, "smlm_pkm_bag: %d threads for %d-chunk rows exceed the kernel's %d", nthr,
                  cpr, kBagMaxThreads);
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
