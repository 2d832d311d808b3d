// Engram n-gram memory (smlm/engram.py): the row indices of every hash head, and the row gather that reads them.
//
//   engram_hash_kernel   NgramHash.forward (smlm/engram.py:60-73): for token t, n-gram order o (n tokens) and hash
//                        head h, x = XOR over i < n of c[t - i] * mult[o, h, i] (64-bit wrap-around products),
//                        x ^= x >> 17 (arithmetic shift), row = (x mod rows, non-negative) + (o * heads + h) * rows.
//                        One thread per (token, lookup); lookups of a token are adjacent in the output.
//   row_gather_kernel    the row lookup of EngramMemory.forward (smlm/engram.py:111-118), F.embedding of the flat
//                        row indices: out[m] = table[rows[m]].  Each thread copies 16 bytes (rows whose width is a
//                        multiple of 16 bytes) or one element; consecutive threads write consecutive bytes of the
//                        output.  A row outside the table gives a NaN output row (no fault), as the value bag does.
#include "pkm_common.h"

namespace smlm {
namespace {

constexpr int kHashThreads = 256;
constexpr int kGatherThreads = 256;
constexpr int kMaxOrders = 4;
constexpr int kMaxOrderLen = 8;

struct HashSpec {
  int n_orders, heads, max_order, history;
  int order[kMaxOrders];
  int64_t rows;
};

__global__ void __launch_bounds__(kHashThreads)
    engram_hash_kernel(const int64_t *__restrict__ c, int64_t T, int64_t c_len, int64_t total,
                       const int64_t *__restrict__ mult, HashSpec spec, int64_t *__restrict__ rows_out) {
  const int lookups = spec.n_orders * spec.heads;
  for (int64_t i = (int64_t)blockIdx.x * kHashThreads + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * kHashThreads) {
    const int j = (int)(i % lookups);
    const int64_t bt = i / lookups;
    const int64_t b = bt / T, t = bt % T;
    const int o = j / spec.heads;
    const int64_t *tok = c + b * c_len + spec.history + t;  // tok[-k] = token t - k
    const int64_t *m = mult + (int64_t)j * spec.max_order;   // mult[o, h, :], j = o * heads + h
    int64_t x = 0;
    for (int k = 0; k < spec.order[o]; ++k) x ^= (int64_t)((uint64_t)tok[-k] * (uint64_t)m[k]);
    x ^= x >> 17;
    int64_t r = x % spec.rows;
    if (r < 0) r += spec.rows;
    rows_out[i] = r + (int64_t)j * spec.rows;
  }
}

template <bool F32, bool VEC>
__global__ void __launch_bounds__(kGatherThreads)
    row_gather_kernel(const int64_t *__restrict__ rows, int64_t total, int per_row, const void *__restrict__ table,
                      int64_t table_rows, int D, void *__restrict__ out) {
  constexpr int EB = F32 ? 4 : 2;                // bytes per element
  constexpr int PER = VEC ? 16 / EB : 1;         // elements per thread
  for (int64_t i = (int64_t)blockIdx.x * kGatherThreads + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * kGatherThreads) {
    const int64_t m = i / per_row;
    const int col = (int)(i % per_row) * PER;
    const int64_t r = rows[m];
    const bool ok = r >= 0 && r < table_rows;
    const int64_t src = (ok ? r : 0) * D + col, dst = m * D + col;
    if constexpr (VEC) {
      const uint32_t nan2 = F32 ? 0x7FC00000u : 0x7FC07FC0u;
      uint4 v = ok ? *(const uint4 *)((const char *)table + src * EB) : uint4{nan2, nan2, nan2, nan2};
      *(uint4 *)((char *)out + dst * EB) = v;
    } else if constexpr (F32) {
      ((float *)out)[dst] = ok ? ((const float *)table)[src] : __builtin_nanf("");
    } else {
      ((uint16_t *)out)[dst] = ok ? ((const uint16_t *)table)[src] : (uint16_t)0x7FC0;
    }
  }
}

int64_t grid_for(int64_t total, int threads) {
  int64_t blocks = (total + threads - 1) / threads;
  return blocks > 65536 ? 65536 : blocks;  // grid-stride beyond
}

}  // namespace
}  // namespace smlm

extern "C" int smlm_engram_hash(const int64_t *c, int64_t B, int64_t T, int64_t c_len, const int64_t *mult,
                                const int *orders, int n_orders, int heads, int max_order, int64_t rows_per_head,
                                int64_t *rows_out, void *stream) {
  using namespace smlm;
  if (!c || !mult || !orders || !rows_out) return fail(SMLM_EINVAL, "smlm_engram_hash: null pointer argument");
  if (n_orders < 1 || n_orders > kMaxOrders || heads < 1 || max_order < 1 || max_order > kMaxOrderLen ||
      rows_per_head < 1 || B < 0 || T < 0)
    return fail(SMLM_EUNSUPPORTED, "smlm_engram_hash: n_orders=%d heads=%d max_order=%d rows=%lld B=%lld T=%lld "
                "(1-%d orders of at most %d tokens)", n_orders, heads, max_order, (long long)rows_per_head,
                (long long)B, (long long)T, kMaxOrders, kMaxOrderLen);
  HashSpec spec{};
  spec.n_orders = n_orders;
  spec.heads = heads;
  spec.max_order = max_order;
  spec.rows = rows_per_head;
  int longest = 0;
  for (int o = 0; o < n_orders; ++o) {
    if (orders[o] < 1 || orders[o] > max_order)
      return fail(SMLM_EINVAL, "smlm_engram_hash: order %d is %d, outside [1, max_order=%d]", o, orders[o],
                  max_order);
    spec.order[o] = orders[o];
    longest = orders[o] > longest ? orders[o] : longest;
  }
  spec.history = longest - 1;
  if (c_len != T + spec.history)
    return fail(SMLM_EINVAL, "smlm_engram_hash: c has %lld columns, expected T + history = %lld", (long long)c_len,
                (long long)(T + spec.history));
  const int64_t total = B * T * n_orders * heads;
  if (total == 0) return SMLM_OK;
  hipLaunchKernelGGL(engram_hash_kernel, dim3((unsigned)grid_for(total, kHashThreads)), dim3(kHashThreads), 0,
                     (hipStream_t)stream, c, T, c_len, total, mult, spec, rows_out);
  return launch_status("smlm_engram_hash");
}

extern "C" int smlm_row_gather(const int64_t *rows, int64_t M, const void *table, int table_dtype,
                               int64_t table_rows, int D, void *out, void *stream) {
  using namespace smlm;
  if (!rows || !table || !out) return fail(SMLM_EINVAL, "smlm_row_gather: null pointer argument");
  if (table_dtype != SMLM_F32 && table_dtype != SMLM_BF16)
    return fail(SMLM_EINVAL, "smlm_row_gather: the table must be SMLM_F32 or SMLM_BF16, got %d", table_dtype);
  if (M < 0 || table_rows < 1 || D < 1)
    return fail(SMLM_EINVAL, "smlm_row_gather: M=%lld table_rows=%lld D=%d", (long long)M, (long long)table_rows, D);
  if (M == 0) return SMLM_OK;
  const bool f32 = table_dtype == SMLM_F32;
  const int per16 = f32 ? 4 : 8;
  const bool vec = D % per16 == 0 && (uintptr_t)table % 16 == 0 && (uintptr_t)out % 16 == 0;
  const int per_row = vec ? D / per16 : D;
  const int64_t total = M * per_row;
  const dim3 grid((unsigned)grid_for(total, kGatherThreads)), block(kGatherThreads);
  hipStream_t s = (hipStream_t)stream;
  if (f32 && vec)
    hipLaunchKernelGGL((row_gather_kernel<true, true>), grid, block, 0, s, rows, total, per_row, table, table_rows, D,
                       out);
  else if (f32)
    hipLaunchKernelGGL((row_gather_kernel<true, false>), grid, block, 0, s, rows, total, per_row, table, table_rows,
                       D, out);
  else if (vec)
    hipLaunchKernelGGL((row_gather_kernel<false, true>), grid, block, 0, s, rows, total, per_row, table, table_rows,
                       D, out);
  else
    hipLaunchKernelGGL((row_gather_kernel<false, false>), grid, block, 0, s, rows, total, per_row, table, table_rows,
                       D, out);
  return launch_status("smlm_row_gather");
}
