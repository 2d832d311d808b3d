// Memory ceilings of the GPU the benchmark runs on, measured by kernels that do nothing but move bytes.  The
// lookup kernels' measured rates are reported against these as well as against the vendor's 8 TB/s.
//   smlm_bench_stream       sequential 16-byte loads and/or stores over one buffer (read, write, copy), every
//                           workgroup striding over the whole buffer with kStreamUnroll accesses in flight per thread;
//   smlm_bench_random_rows  whole rows of `row_bytes` (a multiple of 16) at given int64 row indices, the way the value
//                           gather reads them (row slots x 16-byte chunk columns, coalesced within a row), with no
//                           arithmetic and no output beyond a never-taken store; the launch shape is a parameter
//                           (row slots per workgroup, rows in flight per thread) so the caller can take the best.
// Neither is part of the lookup library: bench.py loads this file's library (libsmlm_bench.so) on its own.
// The loaded data is folded into one word per thread and stored only if it equals a constant no input here makes,
// so the loads cannot be removed and nothing but the buffers is written.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

constexpr int kStreamThreads = 256;
constexpr int kStreamUnroll = 8;
constexpr uint32_t kNever = 0x9E3779B9u;

__device__ __forceinline__ uint32_t fold(const uint4 v) { return v.x ^ v.y ^ v.z ^ v.w; }

// OP 0: read, 1: write, 2: copy.  n16 = buffer size in 16-byte units; the grid strides over it.
template <int OP>
__global__ void __launch_bounds__(kStreamThreads) stream_kernel(const uint4 *__restrict__ src, uint4 *__restrict__ dst,
                                                               int64_t n16, uint32_t *__restrict__ sink) {
  const int64_t step = (int64_t)gridDim.x * kStreamThreads * kStreamUnroll;
  uint32_t acc = 0;
  for (int64_t base = (int64_t)blockIdx.x * kStreamThreads * kStreamUnroll + threadIdx.x; base < n16;
       base += step) {
    uint4 v[kStreamUnroll];
    if constexpr (OP != 1) {
#pragma unroll
      for (int u = 0; u < kStreamUnroll; ++u) {
        const int64_t i = base + (int64_t)u * kStreamThreads;
        v[u] = i < n16 ? src[i] : uint4{0, 0, 0, 0};
      }
    } else {
#pragma unroll
      for (int u = 0; u < kStreamUnroll; ++u) {
        const uint32_t x = (uint32_t)(base + u);
        v[u] = uint4{x, x + 1, x + 2, x + 3};
      }
    }
    if constexpr (OP == 0) {
#pragma unroll
      for (int u = 0; u < kStreamUnroll; ++u) acc ^= fold(v[u]);
    } else {
#pragma unroll
      for (int u = 0; u < kStreamUnroll; ++u) {
        const int64_t i = base + (int64_t)u * kStreamThreads;
        if (i < n16) dst[i] = v[u];
      }
    }
  }
  if (OP == 0 && acc == kNever) sink[0] = acc;
}

// One workgroup reads SLOTS * RPT rows: thread (slot, c) loads chunk c of rows base + slot + u * SLOTS,
// u < RPT, all issued before any is used.  Indices are clamped into [0, rows).
template <int CPR, int SLOTS, int RPT>
__global__ void __launch_bounds__(CPR *SLOTS) random_rows_kernel(const int64_t *__restrict__ idx, int64_t n,
                                                                 const uint8_t *__restrict__ table, int64_t rows,
                                                                 uint32_t *__restrict__ sink) {
  const int tid = threadIdx.x, c = tid % CPR, slot = tid / CPR;
  const int64_t base = (int64_t)blockIdx.x * SLOTS * RPT + slot;
  int64_t off[RPT];
#pragma unroll
  for (int u = 0; u < RPT; ++u) {
    const int64_t j = min(base + (int64_t)u * SLOTS, n - 1);
    const int64_t r = idx[j];
    off[u] = (r < 0 ? 0 : r >= rows ? rows - 1 : r) * (CPR * 16) + c * 16;
  }
  uint4 v[RPT];
#pragma unroll
  for (int u = 0; u < RPT; ++u) v[u] = *(const uint4 *)(table + off[u]);
  uint32_t acc = 0;
#pragma unroll
  for (int u = 0; u < RPT; ++u) acc ^= base + (int64_t)u * SLOTS < n ? fold(v[u]) : 0u;
  if (acc == kNever) sink[0] = acc;
}

template <int CPR, int SLOTS, int RPT>
void launch_rows(const int64_t *idx, int64_t n, const void *table, int64_t rows, uint32_t *sink, hipStream_t s) {
  const int64_t per = (int64_t)SLOTS * RPT;
  hipLaunchKernelGGL((random_rows_kernel<CPR, SLOTS, RPT>), dim3((unsigned)((n + per - 1) / per)), dim3(CPR * SLOTS),
                     0, s, idx, n, (const uint8_t *)table, rows, sink);
}

template <int CPR>
int launch_rows_shape(int shape, const int64_t *idx, int64_t n, const void *table, int64_t rows, uint32_t *sink,
                      hipStream_t s) {
  switch (shape) {
    case 0: launch_rows<CPR, 8, 16>(idx, n, table, rows, sink, s); return 0;   // the value gather's layout
    case 1: launch_rows<CPR, 8, 32>(idx, n, table, rows, sink, s); return 0;
    case 2: launch_rows<CPR, 16, 8>(idx, n, table, rows, sink, s); return 0;
    case 3: launch_rows<CPR, 16, 16>(idx, n, table, rows, sink, s); return 0;
    case 4: launch_rows<CPR, 4, 16>(idx, n, table, rows, sink, s); return 0;
    default: return -1;
  }
}

}  // namespace

// Shapes of smlm_bench_random_rows: 0 .. smlm_bench_random_row_shapes() - 1.
extern "C" int smlm_bench_random_row_shapes() { return 5; }

// (row slots per workgroup, rows in flight per thread) of a shape, as slots * 1000 + rows, or -1.
extern "C" int smlm_bench_random_row_shape(int shape) {
  static const int t[] = {8016, 8032, 16008, 16016, 4016};
  return shape >= 0 && shape < 5 ? t[shape] : -1;
}

// op 0: read `bytes` at src; 1: write them at dst; 2: copy src to dst.  bytes % 16 == 0, 16-byte aligned buffers.
extern "C" int smlm_bench_stream(int op, const void *src, void *dst, int64_t bytes, int grid, void *sink,
                                 void *stream) {
  if (bytes <= 0 || bytes % 16 || grid < 1 || !sink || (op != 1 && !src) || (op != 0 && !dst) ||
      ((uintptr_t)src | (uintptr_t)dst) % 16)
    return -1;
  hipStream_t s = (hipStream_t)stream;
  const int64_t n16 = bytes / 16;
  const uint4 *a = (const uint4 *)src;
  uint4 *b = (uint4 *)dst;
  uint32_t *k = (uint32_t *)sink;
  switch (op) {
    case 0: hipLaunchKernelGGL(stream_kernel<0>, dim3(grid), dim3(kStreamThreads), 0, s, a, b, n16, k); break;
    case 1: hipLaunchKernelGGL(stream_kernel<1>, dim3(grid), dim3(kStreamThreads), 0, s, a, b, n16, k); break;
    case 2: hipLaunchKernelGGL(stream_kernel<2>, dim3(grid), dim3(kStreamThreads), 0, s, a, b, n16, k); break;
    default: return -1;
  }
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

// Read the rows idx[0..n) (int64, clamped into [0, rows)) of a table of `rows` rows of row_bytes (384 or 768).
extern "C" int smlm_bench_random_rows(const int64_t *idx, int64_t n, const void *table, int64_t rows, int row_bytes,
                                      int shape, void *sink, void *stream) {
  if (!idx || !table || !sink || n < 1 || rows < 1 || (uintptr_t)table % 16 || (uintptr_t)idx % 8) return -1;
  hipStream_t s = (hipStream_t)stream;
  int rc;
  if (row_bytes == 384) rc = launch_rows_shape<24>(shape, idx, n, table, rows, (uint32_t *)sink, s);
  else if (row_bytes == 768) rc = launch_rows_shape<48>(shape, idx, n, table, rows, (uint32_t *)sink, s);
  else return -1;
  if (rc) return rc;
  return hipGetLastError() == hipSuccess ? 0 : -2;
}
