// Row-sparse value-bag backward in a fixed order, through one sort of all the lookups by table row (the grouping of
// the reference's bag_backward_rows, smlm/kernels.py:34-88, which sorts the lookups and adds each row's run):
//   acc[idx[n,k], :] += w[n,k] * grad_out[n, :],  touched[idx[n,k]] = 1,  gw[n,k] = grad_out[n, :] . table[idx[n,k], :]
//
//   1. keys_kernel: (row, lookup) pairs for the L = N K lookups, an index outside the table keyed past every row;
//   2. a stable radix sort of the pairs by row (rocPRIM), so each row's lookups form one run in lookup order;
//   3. runs_kernel: one wavefront per chunk of 64 sorted lookups walks its segments of equal rows (a few at a time,
//      their table, accumulator and first gradient rows in flight together): one table-row read per segment, the
//      per-sample-weight gradient of each lookup (gradient rows loaded 8 lookups at a time), and the segment's sum
//      of w x g in registers, added in lookup order.  A run that starts and ends in the chunk updates its
//      accumulator row with a plain read-add-write (the row has no other writer); a segment at a chunk edge that
//      continues into the neighbouring chunk leaves its sum in a per-chunk partial;
//   4. group_sums_kernel: the partials of each group of 32 chunks that lies inside one run, summed in a fixed order;
//   5. cross_runs_kernel: for each run that crosses chunk edges, a workgroup finds the run's end in the sorted keys
//      (a 64-lane search), adds the partials of its chunks (whole groups by their sums) in a fixed order and updates
//      the row once.
// Every accumulator row has one writer and every sum a fixed order, so the result does not depend on scheduling
// (the atomic form in pkm_train.hip is faster to start but pays contention on rows read by many tokens).
#include <cstring>
#include <rocprim/device/device_radix_sort.hpp>

#include "pkm_common.h"

namespace smlm {
namespace {

constexpr int kRunThreads = 256;                    // 4 wavefronts, one sorted chunk each
constexpr int kChunk = kWave;                       // sorted lookups per wavefront
constexpr int kChunksPerBlock = kRunThreads / kWave;
constexpr int kCrossWaves = 4;                      // wavefronts of a crossing-run workgroup
constexpr int kGroup = 32;                          // chunks per group sum (runs spanning whole groups)
constexpr int kSegsInFlight = 3;                    // segments whose rows are loaded together
constexpr int kLookAhead = 8;                       // lookups of a segment whose gradient rows are loaded together
constexpr int kMaxDSorted = 512;
// the stable radix sort in onesweep passes (one per 8 key bits) at every size: rocPRIM's default sorts fewer than
// 2^20 items by block sort + merge passes (18 launches at 524,288 lookups, ~125 us against ~3 radix passes).  The
// passes: 1024 threads x 4 keys per block, ranks by the match algorithm (timing probe of 524,288 21-bit keys, sorted
// and stable each time: 59 us, against 96 us for rocPRIM's onesweep defaults; 65-70 us at 2-3 or 8 keys per thread,
// 512 threads 68 us, 7-bit digits 60 us, 11-bit digits 67-85 us; 8-bit digits above 4 keys per thread at 512 or 1024
// threads need more than the 160 KB of LDS without the match ranks)
using SortConfig = rocprim::radix_sort_config<
    rocprim::default_config, rocprim::default_config,
    rocprim::radix_sort_onesweep_config<rocprim::kernel_config<1024, 4>, rocprim::kernel_config<1024, 4>, 8,
                                        rocprim::block_radix_rank_algorithm::match>,
    0>;

template <bool F32>
__device__ __forceinline__ float table_value(const void *table, int64_t i) {
  if constexpr (F32) return ((const float *)table)[i];
  else return bf16_bits_to_f32(((const uint16_t *)table)[i]);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = kWave / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

__global__ void __launch_bounds__(256) keys_kernel(const int64_t *__restrict__ idx, int64_t L, uint32_t rows,
                                                   uint32_t *__restrict__ keys, uint32_t *__restrict__ vals) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < L) {
    const int64_t r = idx[i];
    keys[i] = r >= 0 && r < (int64_t)rows ? (uint32_t)r : rows;   // outside the table: after every row
    vals[i] = (uint32_t)i;
  }
}

// lane l holds columns l, l + 64, .. (CPL of them) of a row
template <bool TABLE_F32, int CPL>
__global__ void __launch_bounds__(kRunThreads)
    runs_kernel(const float *__restrict__ grad_out, const float *__restrict__ w, int K, const void *__restrict__ table,
                uint32_t rows, int D, const uint32_t *__restrict__ keys, const uint32_t *__restrict__ vals, int64_t L,
                float *__restrict__ acc, uint8_t *__restrict__ touched, float *__restrict__ gw,
                float *__restrict__ partial, uint8_t *__restrict__ cross) {
  const int lane = lane_id();
  const int64_t c = (int64_t)blockIdx.x * kChunksPerBlock + threadIdx.x / kWave;
  const int64_t p0 = c * kChunk;
  if (p0 >= L) return;                              // wavefront-uniform; this kernel has no barrier
  const int64_t p = p0 + lane;
  const bool inb = p < L;
  const uint32_t key = inb ? keys[p] : rows;
  const uint32_t v = inb ? vals[p] : 0u;
  const bool valid = key < rows;                    // valid keys precede the rest of the chunk
  if (inb && !valid) gw[v] = __builtin_nanf("");    // an index outside the table: NaN weight gradient, no update
  const uint32_t before = p0 > 0 ? keys[p0 - 1] : rows;
  const uint32_t after = p0 + kChunk < L ? keys[p0 + kChunk] : rows;
  const uint32_t prev = (uint32_t)__shfl_up((int)key, 1, kWave);
  uint64_t heads = __builtin_amdgcn_ballot_w64(valid && (lane == 0 || prev != key));
  const int nvalid = __popcll(__builtin_amdgcn_ballot_w64(valid));
  bool crosses = false;

  while (heads) {
    int h[kSegsInFlight], end[kSegsInFlight], mode[kSegsInFlight];   // mode 0: whole run, 1: continues a run, 2: starts one
    uint32_t r[kSegsInFlight];
    float tv[kSegsInFlight][CPL], av[kSegsInFlight][CPL], g0[kSegsInFlight][CPL];
#pragma unroll
    for (int u = 0; u < kSegsInFlight; ++u) {
      h[u] = heads ? __builtin_ctzll(heads) : kWave;
      heads = heads ? heads & (heads - 1) : 0;
    }
#pragma unroll
    for (int u = 0; u < kSegsInFlight; ++u) {
      const int nxt = u + 1 < kSegsInFlight ? h[u + 1] : (heads ? __builtin_ctzll(heads) : kWave);
      end[u] = nxt < kWave ? nxt : nvalid;
      const bool live = h[u] < kWave;
      r[u] = live ? (uint32_t)__builtin_amdgcn_readlane((int)key, h[u]) : 0u;
      const bool from_prev = h[u] == 0 && before == r[u];
      const bool to_next = end[u] == kChunk && after == r[u];
      mode[u] = from_prev ? 1 : to_next ? 2 : 0;
      const int64_t n0 = live ? (int64_t)((uint32_t)__builtin_amdgcn_readlane((int)v, h[u]) / (uint32_t)K) : 0;
#pragma unroll
      for (int e = 0; e < CPL; ++e) {
        const int d = lane + kWave * e;
        const bool col = live && d < D;
        tv[u][e] = col ? table_value<TABLE_F32>(table, (int64_t)r[u] * D + d) : 0.f;
        av[u][e] = col && mode[u] == 0 ? acc[(int64_t)r[u] * D + d] : 0.f;
        g0[u][e] = col ? grad_out[n0 * D + d] : 0.f;
      }
    }
#pragma unroll
    for (int u = 0; u < kSegsInFlight; ++u) {
      if (h[u] >= kWave) break;                     // wavefront-uniform
      float s[CPL];
#pragma unroll
      for (int e = 0; e < CPL; ++e) s[e] = 0.f;
      // the segment's first lookup (its gradient row loaded with the segment's rows), then the rest kLookAhead at
      // a time, their gradient rows and weights loaded together (a hot row's segment fills whole chunks: one memory
      // round trip per group); the products in lookup order
      {
        const uint32_t vh = (uint32_t)__builtin_amdgcn_readlane((int)v, h[u]);
        const float wh = w[vh];
        float dot = 0.f;
#pragma unroll
        for (int e = 0; e < CPL; ++e) {
          dot = fmaf(g0[u][e], tv[u][e], dot);
          s[e] = s[e] + wh * g0[u][e];
        }
        dot = wave_sum(dot);
        if (lane == 0) gw[vh] = dot;
      }
      for (int j0 = h[u] + 1; j0 < end[u]; j0 += kLookAhead) {
        const int cnt = end[u] - j0 < kLookAhead ? end[u] - j0 : kLookAhead;   // wavefront-uniform
        uint32_t vv[kLookAhead];
        float wv[kLookAhead], gv[kLookAhead][CPL];
#pragma unroll
        for (int q = 0; q < kLookAhead; ++q) {
          if (q >= cnt) break;
          vv[q] = (uint32_t)__builtin_amdgcn_readlane((int)v, j0 + q);
          const int64_t nq = (int64_t)(vv[q] / (uint32_t)K);
          wv[q] = w[vv[q]];
#pragma unroll
          for (int e = 0; e < CPL; ++e) {
            const int d = lane + kWave * e;
            gv[q][e] = d < D ? grad_out[nq * D + d] : 0.f;
          }
        }
#pragma unroll
        for (int q = 0; q < kLookAhead; ++q) {
          if (q >= cnt) break;
          float dot = 0.f;
#pragma unroll
          for (int e = 0; e < CPL; ++e) {
            dot = fmaf(gv[q][e], tv[u][e], dot);
            s[e] = s[e] + wv[q] * gv[q][e];
          }
          dot = wave_sum(dot);
          if (lane == 0) gw[vv[q]] = dot;
        }
      }
      const int64_t ro = (int64_t)r[u] * D;
      if (mode[u] == 0) {
#pragma unroll
        for (int e = 0; e < CPL; ++e) {
          const int d = lane + kWave * e;
          if (d < D) acc[ro + d] = av[u][e] + s[e];
        }
        if (lane == 0) touched[r[u]] = 1;
      } else {
        float *dst = partial + (2 * c + (mode[u] == 1 ? 0 : 1)) * (int64_t)D;
#pragma unroll
        for (int e = 0; e < CPL; ++e) {
          const int d = lane + kWave * e;
          if (d < D) dst[d] = s[e];
        }
        crosses = crosses || mode[u] == 2;
      }
    }
  }
  if (lane == 0) cross[c] = crosses ? 1 : 0;
}

// The last sorted position holding key r, for a run known to cover position lo: 64 lanes probe at once, first
// at exponentially spaced positions past lo, then 64 evenly spaced positions of the bracket found, so a run of
// length n costs about log_64(n) + 1 dependent rounds of loads.  Every lane returns the same position.
__device__ __forceinline__ int64_t run_last(const uint32_t *__restrict__ keys, int64_t L, uint32_t r, int64_t lo) {
  const int lane = lane_id();
  // round 1: positions lo + 2^lane - 1 (lane 0: lo itself)
  const int64_t step = lane < 62 ? ((int64_t)1 << lane) - 1 : L;
  const int64_t pos = lo + step < L ? lo + step : L - 1;
  const bool in_run = keys[pos] == r;
  // the positions covered are a prefix of the lanes (keys are sorted): the last such lane brackets the end
  const uint64_t cov = __builtin_amdgcn_ballot_w64(in_run && (lane == 0 || lo + step < L));
  int last = 63 - __builtin_clzll(cov);                          // lane 0 always covers lo
  int64_t a = lo + (last < 62 ? ((int64_t)1 << last) - 1 : 0);  // known in the run
  int64_t b = last + 1 < 62 ? lo + ((int64_t)1 << (last + 1)) - 1 : L;   // known past it (or L)
  if (b > L) b = L;
  while (b - a > 1) {                                            // 64-way narrowing: a in the run, b past it
    const int64_t span = b - a;
    const int64_t q = a + 1 + (span - 1) * lane / kWave;         // strictly inside (a, b), nondecreasing in lane
    const bool hit = q < b && keys[q] == r;
    const uint64_t hits = __builtin_amdgcn_ballot_w64(hit);
    if (hits == 0) break;                                        // a + 1 is past the run: a is its end
    const int hl = 63 - __builtin_clzll(hits);
    const int64_t na = a + 1 + (span - 1) * hl / kWave;
    const int64_t nb = hl + 1 < kWave ? a + 1 + (span - 1) * (hl + 1) / kWave : b;
    a = na;
    b = nb > a ? nb : a + 1;
  }
  return a;
}

// Rows first .. last of base (row i at i * stride), wavefront `wave` of kCrossWaves taking rows first + wave,
// first + wave + kCrossWaves, .. with 8 loads in flight, added to s in that order.
template <int CPL>
__device__ __forceinline__ void add_rows(const float *__restrict__ base, int64_t stride, int64_t first, int64_t last,
                                         int D, int wave, int lane, float (&s)[CPL]) {
  for (int64_t i0 = first + wave; i0 <= last; i0 += kCrossWaves * 8) {
    float pv[8][CPL];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int64_t i = i0 + (int64_t)q * kCrossWaves;
#pragma unroll
      for (int e = 0; e < CPL; ++e) {
        const int d = lane + kWave * e;
        pv[q][e] = i <= last && d < D ? base[i * stride + d] : 0.f;
      }
    }
#pragma unroll
    for (int q = 0; q < 8; ++q)
#pragma unroll
      for (int e = 0; e < CPL; ++e) s[e] += pv[q][e];
  }
}

// One workgroup per group of kGroup chunks that lies inside one run with the run going on at both sides (its key
// at the positions just before and just after the group): the group's chunks each hold one segment of that run,
// whose sum is their slot-0 partial; their sum, in the order of add_rows and then wavefront order, is the group's.
// A hot row's run of hundreds of chunks then costs its crossing workgroup a few dozen loads instead of one per chunk.
template <int CPL>
__global__ void __launch_bounds__(kCrossWaves * kWave)
    group_sums_kernel(const uint32_t *__restrict__ keys, int64_t L, uint32_t rows, int D,
                      const float *__restrict__ partial, float *__restrict__ gsum) {
  __shared__ float sSum[kCrossWaves][CPL * kWave];
  const int64_t g = blockIdx.x;
  const int64_t p0 = g * kGroup * kChunk, p1 = p0 + kGroup * kChunk;   // the group's positions [p0, p1)
  if (p0 == 0 || p1 >= L) return;                   // workgroup-uniform, before the barrier
  const uint32_t r = keys[p0];
  if (r >= rows || keys[p0 - 1] != r || keys[p1 - 1] != r || keys[p1] != r) return;
  const int lane = lane_id(), wave = threadIdx.x / kWave;
  float s[CPL];
#pragma unroll
  for (int e = 0; e < CPL; ++e) s[e] = 0.f;
  add_rows<CPL>(partial, 2 * (int64_t)D, g * kGroup, g * kGroup + kGroup - 1, D, wave, lane, s);
#pragma unroll
  for (int e = 0; e < CPL; ++e) sSum[wave][e * kWave + lane] = s[e];
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int e = 0; e < CPL; ++e) {
    const int d = lane + kWave * e;
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < kCrossWaves; ++i) t += sSum[i][e * kWave + lane];
    if (d < D) gsum[g * D + d] = t;
  }
}

// One workgroup per chunk; a chunk whose last segment starts a run that continues into the next chunk (cross[c])
// adds the run's partial sums: its own (slot 1), then the continuation chunks' (slot 0) and whole groups' sums
// (add_rows: wavefront i taking every fourth row, 8 loads in flight), the four sums added in wavefront order
// through LDS.
template <int CPL>
__global__ void __launch_bounds__(kCrossWaves * kWave)
    cross_runs_kernel(const uint32_t *__restrict__ keys, int64_t L, int D, const float *__restrict__ partial,
                      const float *__restrict__ gsum, const uint8_t *__restrict__ cross, float *__restrict__ acc,
                      uint8_t *__restrict__ touched) {
  __shared__ float sSum[kCrossWaves][CPL * kWave];
  const int64_t c = blockIdx.x;
  if (!cross[c]) return;                            // workgroup-uniform, before the barrier
  const int lane = lane_id(), wave = threadIdx.x / kWave;
  const uint32_t r = keys[c * kChunk + kChunk - 1];  // the run fills chunk c to its end
  const int64_t last = run_last(keys, L, r, c * kChunk + kChunk - 1);
  const int64_t c_last = last / kChunk;             // the run's last chunk (> c)
  float s[CPL];
#pragma unroll
  for (int e = 0; e < CPL; ++e) s[e] = 0.f;
  // the continuation chunks c + 1 .. c_last: whole groups of kGroup chunks strictly before c_last by their group
  // sums (group_sums_kernel wrote every such group: the run covers it and the positions on both sides of it), the
  // chunks before and after them one by one
  const int64_t g_lo = (c + 1 + kGroup - 1) / kGroup, g_hi = c_last / kGroup - 1;
  if (g_lo <= g_hi) {
    add_rows<CPL>(partial, 2 * (int64_t)D, c + 1, g_lo * kGroup - 1, D, wave, lane, s);
    add_rows<CPL>(gsum, D, g_lo, g_hi, D, wave, lane, s);
    add_rows<CPL>(partial, 2 * (int64_t)D, (g_hi + 1) * kGroup, c_last, D, wave, lane, s);
  } else {
    add_rows<CPL>(partial, 2 * (int64_t)D, c + 1, c_last, D, wave, lane, s);
  }
#pragma unroll
  for (int e = 0; e < CPL; ++e) sSum[wave][e * kWave + lane] = s[e];
  __syncthreads();
  if (wave != 0) return;
  const int64_t ro = (int64_t)r * D;
#pragma unroll
  for (int e = 0; e < CPL; ++e) {
    const int d = lane + kWave * e;
    float t = d < D ? partial[(2 * c + 1) * (int64_t)D + d] : 0.f;   // the run's first chunk, then the rest
#pragma unroll
    for (int i = 0; i < kCrossWaves; ++i) t += sSum[i][e * kWave + lane];
    if (d < D) acc[ro + d] += t;
  }
  if (lane == 0) touched[r] = 1;
}

// workspace: keys and values in / out, partials, group sums, cross flags, the sort's own storage (each 256-byte
// aligned)
struct SortedLayout {
  size_t keys_in, vals_in, keys_out, vals_out, partial, gsum, cross, sort_tmp, sort_bytes, total;
};

size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

int end_bit_for(uint32_t rows) { return 32 - __builtin_clz(rows); }   // the keys go up to rows (outside the table)

int sorted_layout(int64_t L, int64_t rows, int D, SortedLayout &lay) {
  const size_t l4 = align256((size_t)L * 4), nchunks = (size_t)((L + kChunk - 1) / kChunk);
  lay.keys_in = 0;
  lay.vals_in = lay.keys_in + l4;
  lay.keys_out = lay.vals_in + l4;
  lay.vals_out = lay.keys_out + l4;
  lay.partial = lay.vals_out + l4;
  lay.gsum = lay.partial + align256(nchunks * 2 * (size_t)D * 4);
  lay.cross = lay.gsum + align256((nchunks + kGroup - 1) / kGroup * (size_t)D * 4);
  lay.sort_tmp = lay.cross + align256(nchunks);
  size_t bytes = 0;
  const hipError_t e = rocprim::radix_sort_pairs<SortConfig>(nullptr, bytes, (const uint32_t *)nullptr, (uint32_t *)nullptr,
                                                 (const uint32_t *)nullptr, (uint32_t *)nullptr, (unsigned)L, 0,
                                                 end_bit_for((uint32_t)rows), (hipStream_t)0);
  if (e != hipSuccess) return fail(SMLM_EHIP, "smlm_bag_backward_sorted: sort storage query: %s", hipGetErrorString(e));
  lay.sort_bytes = align256(bytes);
  lay.total = lay.sort_tmp + lay.sort_bytes;
  return SMLM_OK;
}

int check_sorted_shape(const char *what, int64_t N, int K, int64_t rows, int D) {
  if (N < 0 || K < 1 || rows < 1 || D < 1 || D > kMaxDSorted)
    return fail(SMLM_EUNSUPPORTED, "%s: N=%lld K=%d rows=%lld D=%d (1 <= D <= %d)", what, (long long)N, K,
                (long long)rows, D, kMaxDSorted);
  if (rows >= 0xFFFFFFFFLL || (int64_t)N * K >= 0x7FFFFFFFLL)
    return fail(SMLM_EUNSUPPORTED, "%s: rows=%lld and N*K=%lld must stay below 2^32 - 1 and 2^31 - 1", what,
                (long long)rows, (long long)((int64_t)N * K));
  return SMLM_OK;
}

template <int CPL>
void launch_runs(const float *grad_out, const float *w, int K, const void *table, bool f32, uint32_t rows, int D,
                 const uint32_t *keys, const uint32_t *vals, int64_t L, float *acc, uint8_t *touched, float *gw,
                 float *partial, float *gsum, uint8_t *cross, hipStream_t s) {
  const int64_t nchunks = (L + kChunk - 1) / kChunk;
  const dim3 grid((unsigned)((nchunks + kChunksPerBlock - 1) / kChunksPerBlock)), block(kRunThreads);
  if (f32)
    hipLaunchKernelGGL((runs_kernel<true, CPL>), grid, block, 0, s, grad_out, w, K, table, rows, D, keys, vals, L, acc,
                       touched, gw, partial, cross);
  else
    hipLaunchKernelGGL((runs_kernel<false, CPL>), grid, block, 0, s, grad_out, w, K, table, rows, D, keys, vals, L,
                       acc, touched, gw, partial, cross);
  hipLaunchKernelGGL((group_sums_kernel<CPL>), dim3((unsigned)((nchunks + kGroup - 1) / kGroup)),
                     dim3(kCrossWaves * kWave), 0, s, keys, L, rows, D, (const float *)partial, gsum);
  hipLaunchKernelGGL((cross_runs_kernel<CPL>), dim3((unsigned)nchunks), dim3(kCrossWaves * kWave), 0, s, keys, L, D,
                     (const float *)partial, (const float *)gsum, (const uint8_t *)cross, acc, touched);
}

}  // namespace
}  // namespace smlm

extern "C" int smlm_bag_backward_sorted_workspace(int64_t N, int K, int64_t rows, int D, size_t *bytes) {
  using namespace smlm;
  if (!bytes) return fail(SMLM_EINVAL, "smlm_bag_backward_sorted_workspace: null bytes pointer");
  const int rc = check_sorted_shape("smlm_bag_backward_sorted_workspace", N, K, rows, D);
  if (rc != SMLM_OK) return rc;
  SortedLayout lay;
  const int64_t L = N * K;
  if (L == 0) {
    *bytes = 0;
    return SMLM_OK;
  }
  const int lr = sorted_layout(L, rows, D, lay);
  if (lr != SMLM_OK) return lr;
  *bytes = lay.total;
  return SMLM_OK;
}

extern "C" int smlm_bag_backward_sorted(const float *grad_out, const int64_t *idx, const float *w, int64_t N, int K,
                                        const void *table, int table_dtype, int64_t rows, int D, float *acc,
                                        uint8_t *touched, float *gw, void *workspace, size_t workspace_bytes,
                                        void *stream) {
  using namespace smlm;
  if (!grad_out || !idx || !w || !table || !acc || !touched || !gw)
    return fail(SMLM_EINVAL, "smlm_bag_backward_sorted: null pointer argument");
  if (table_dtype != SMLM_F32 && table_dtype != SMLM_BF16)
    return fail(SMLM_EINVAL, "smlm_bag_backward_sorted: the table must be SMLM_F32 or SMLM_BF16, got %d",
                table_dtype);
  const int rc = check_sorted_shape("smlm_bag_backward_sorted", N, K, rows, D);
  if (rc != SMLM_OK) return rc;
  const int64_t L = N * K;
  if (L == 0) return SMLM_OK;
  SortedLayout lay;
  const int lr = sorted_layout(L, rows, D, lay);
  if (lr != SMLM_OK) return lr;
  if (!workspace || workspace_bytes < lay.total || (uintptr_t)workspace % 256)
    return fail(SMLM_EINVAL, "smlm_bag_backward_sorted: workspace of %zu bytes (256-byte aligned) needed, got %zu",
                lay.total, workspace ? workspace_bytes : (size_t)0);
  hipStream_t s = (hipStream_t)stream;
  unsigned char *ws = (unsigned char *)workspace;
  uint32_t *keys_in = (uint32_t *)(ws + lay.keys_in), *vals_in = (uint32_t *)(ws + lay.vals_in);
  uint32_t *keys = (uint32_t *)(ws + lay.keys_out), *vals = (uint32_t *)(ws + lay.vals_out);
  float *partial = (float *)(ws + lay.partial), *gsum = (float *)(ws + lay.gsum);
  uint8_t *cross = ws + lay.cross;
  hipLaunchKernelGGL(keys_kernel, dim3((unsigned)((L + 255) / 256)), dim3(256), 0, s, idx, L, (uint32_t)rows,
                     keys_in, vals_in);
  size_t sort_bytes = lay.sort_bytes;
  const hipError_t e = rocprim::radix_sort_pairs<SortConfig>(ws + lay.sort_tmp, sort_bytes, keys_in, keys, vals_in, vals,
                                                 (unsigned)L, 0, end_bit_for((uint32_t)rows), s);
  if (e != hipSuccess) return fail(SMLM_EHIP, "smlm_bag_backward_sorted: sort: %s", hipGetErrorString(e));
  const bool f32 = table_dtype == SMLM_F32;
  const uint32_t r32 = (uint32_t)rows;
#define SMLM_RUNS(CPL)                                                                                          \
  launch_runs<CPL>(grad_out, w, K, table, f32, r32, D, keys, vals, L, acc, touched, gw, partial, gsum, cross, s)
  if (D <= 128) SMLM_RUNS(2);
  else if (D <= 256) SMLM_RUNS(4);
  else if (D <= 384) SMLM_RUNS(6);
  else SMLM_RUNS(8);
#undef SMLM_RUNS
  return launch_status("smlm_bag_backward_sorted");
}
