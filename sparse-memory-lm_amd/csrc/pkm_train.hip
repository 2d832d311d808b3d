// Training side of the lookup (the gradients of the selection and of the value bag, and the lazy row Adam of the
// value table):
//
//   select_backward_kernel   PKSelect.backward (smlm/kernels.py:253-266): the softmax backward of each head's knn
//                            weights plus the scores' own gradient, rounded to the scores' dtype, scattered into
//                            dense (N, H, NK) gradients of both halves (sums per sub-key in fp32, in selection
//                            order, rounded once).  One wavefront per (token, head): the two dense rows are
//                            composed in the wavefront's LDS, 64 sixteen-byte chunks at a time (zeros, then the
//                            merged sum of each selected sub-key), and each chunk is written to memory once.
//   bag_backward_kernel      the row-sparse bag backward (smlm/kernels.py:1-104, smlm/sparse_values.py:94-113):
//                            acc[idx[n,k]] += w[n,k] * g[n], touched[idx[n,k]] = 1, and the per-sample-weight
//                            gradient gw[n,k] = g[n] . table[idx[n,k]].  One workgroup per token, a wavefront per
//                            lookup with its row's loads in flight for 4 lookups at a time; the accumulator rows
//                            take hardware fp32 atomic adds (lane l owns columns l, l + 64, ...: each atomic
//                            instruction covers 256 contiguous bytes), so rows read by several lookups need no
//                            sort (the reference sorts the lookups and adds runs, with atomics at the borders).
//                            This is the atomic form; the ordered form, sorted by row with one writer per row
//                            and a fixed order of additions, is smlm_bag_backward_sorted (pkm_train_sorted.hip).
//   lazy_adam_kernel         the lazy Adam step of LazyRowAdam on the rows flagged in `touched` (smlm/kernels.py:
//                            380-515): fp32 moments, or bf16 moments, or int8 companded moments with fp32 row
//                            scales; afterwards the rows' accumulator is zero and their flag cleared.  One
//                            wavefront per row; untouched rows cost one byte read.  No multiply-add contraction in
//                            this file: the update is evaluated in the reference's operation order (its compact
//                            kernel is compiled with fp fusion off), with IEEE division and square root.
#include <type_traits>

#include "pkm_common.h"

#pragma clang fp contract(off)

namespace smlm {
namespace {

constexpr int kTrainThreads = 256;
constexpr int kTrainWaves = kTrainThreads / kWave;
constexpr int kMaxD = 512;                  // columns per row: lane l owns l, l + 64, ... (at most 8 each)
constexpr int kBagInFlight = 4;             // lookups per wavefront whose row loads are issued together

__device__ __forceinline__ float wave_sum_f32(float v) {
  for (int o = kWave / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}
__device__ __forceinline__ float wave_max_f32(float v) {
  for (int o = kWave / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

template <bool F32>
__device__ __forceinline__ float to_dtype(float x) {
  return F32 ? x : round_bf16(x);
}

// ---------------------------------------------------------------------------------------------------------------
template <bool F32>
__global__ void __launch_bounds__(kTrainThreads)
    select_backward_kernel(const int64_t *__restrict__ idx, const float *__restrict__ w, const void *__restrict__ g_scores,
                           const float *__restrict__ g_w, int64_t rows, int NK, int knn, void *__restrict__ ds1,
                           void *__restrict__ ds2) {
  const int lane = lane_id();
  const int64_t row = (int64_t)blockIdx.x * kTrainWaves + threadIdx.x / kWave;  // (n, h)
  if (row >= rows) return;                                                       // wavefront-uniform
  // selected entry j = lane + 64 r (r < 2: knn <= 128)
  bool have[2];
  int64_t ix[2];
  float wk[2], dl[2];
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int j = lane + r * kWave;
    have[r] = j < knn;
    const int64_t o = row * knn + (have[r] ? j : 0);
    ix[r] = have[r] ? idx[o] : 0;
    wk[r] = have[r] ? w[o] : 0.f;
    dl[r] = 0.f;
  }
  if (g_w) {
    float gw[2];
#pragma unroll
    for (int r = 0; r < 2; ++r) gw[r] = have[r] ? g_w[row * knn + lane + r * kWave] : 0.f;
    const float s = wave_sum_f32(wk[0] * gw[0] + wk[1] * gw[1]);
#pragma unroll
    for (int r = 0; r < 2; ++r) dl[r] = wk[r] * (gw[r] - s);
  }
  if (g_scores) {
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int64_t o = row * knn + lane + r * kWave;
      const float gs = !have[r] ? 0.f
                       : F32 ? ((const float *)g_scores)[o]
                             : bf16_bits_to_f32(((const uint16_t *)g_scores)[o]);
      dl[r] = dl[r] + gs;
    }
  }
  float ds[2];
  int i1[2], i2[2];
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    ds[r] = to_dtype<F32>(dl[r]);
    i1[r] = (int)(ix[r] / NK);
    i2[r] = (int)(ix[r] % NK);
  }

  // per sub-key: the sum of its selected pairs' gradients in selection order (every occurrence holds the full sum;
  // the first occurrence of each sub-key is the one that writes it)
  float sum1[2] = {0.f, 0.f}, sum2[2] = {0.f, 0.f};
  bool first1[2] = {have[0], have[1]}, first2[2] = {have[0], have[1]};
  for (int j = 0; j < knn; ++j) {
    const int rj = j / kWave, lj = j % kWave;  // wavefront-uniform
    const int j1 = __builtin_amdgcn_readlane(rj ? i1[1] : i1[0], lj);
    const int j2 = __builtin_amdgcn_readlane(rj ? i2[1] : i2[0], lj);
    const float dj = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, rj ? ds[1] : ds[0]),
                                                                         lj));
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int me = lane + r * kWave;
      if (j1 == i1[r]) {
        sum1[r] = sum1[r] + dj;
        if (j < me) first1[r] = false;
      }
      if (j2 == i2[r]) {
        sum2[r] = sum2[r] + dj;
        if (j < me) first2[r] = false;
      }
    }
  }
  // an index outside [0, NK^2) (not a selection's output) writes nothing
  bool w1[2], w2[2];
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    w1[r] = first1[r] && (unsigned)i1[r] < (unsigned)NK && ix[r] >= 0;
    w2[r] = first2[r] && (unsigned)i2[r] < (unsigned)NK && ix[r] >= 0;
  }
  constexpr int EPV = F32 ? 4 : 8;            // elements per 16 bytes
  char *r1 = (char *)ds1 + row * (int64_t)NK * (F32 ? 4 : 2);
  char *r2 = (char *)ds2 + row * (int64_t)NK * (F32 ? 4 : 2);
  if (NK % EPV == 0) {
    // each 16-byte chunk of both rows written once, with the merged sums of its selected sub-keys in place: the rows
    // are composed in this wavefront's LDS, 64 chunks of each at a time (zeros, then the sums), and streamed to
    // memory (non-temporal, 2 x NK per row, written once)
    typedef unsigned u32x4z __attribute__((ext_vector_type(4)));
    __shared__ u32x4z stage[kTrainWaves][2][kWave];
    u32x4z *st1 = stage[threadIdx.x / kWave][0], *st2 = stage[threadIdx.x / kWave][1];
    const int chunks = NK / EPV;
    for (int cb = 0; cb < chunks; cb += kWave) {
      st1[lane] = u32x4z{0u, 0u, 0u, 0u};
      st2[lane] = u32x4z{0u, 0u, 0u, 0u};
      wave_lds_sync();
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const int e1 = i1[r] - cb * EPV, e2 = i2[r] - cb * EPV;  // element within this pass's 64 chunks
        if (w1[r] && (unsigned)e1 < (unsigned)(kWave * EPV)) {
          if constexpr (F32) ((float *)st1)[e1] = sum1[r];
          else ((uint16_t *)st1)[e1] = (uint16_t)bf16_bits_rtne(sum1[r]);
        }
        if (w2[r] && (unsigned)e2 < (unsigned)(kWave * EPV)) {
          if constexpr (F32) ((float *)st2)[e2] = sum2[r];
          else ((uint16_t *)st2)[e2] = (uint16_t)bf16_bits_rtne(sum2[r]);
        }
      }
      wave_lds_sync();
      if (cb + lane < chunks) {
        __builtin_nontemporal_store(st1[lane], (u32x4z *)(r1 + (int64_t)(cb + lane) * 16));
        __builtin_nontemporal_store(st2[lane], (u32x4z *)(r2 + (int64_t)(cb + lane) * 16));
      }
      wave_lds_sync();
    }
    return;
  }
  // rows that are not whole 16-byte chunks: zeros element by element, every zero store acknowledged, then the sums
  for (int k = lane; k < NK; k += kWave) {
    if constexpr (F32) {
      ((float *)r1)[k] = 0.f;
      ((float *)r2)[k] = 0.f;
    } else {
      ((uint16_t *)r1)[k] = 0;
      ((uint16_t *)r2)[k] = 0;
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_s_waitcnt(0);
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    if constexpr (F32) {
      if (w1[r]) ((float *)r1)[i1[r]] = sum1[r];
      if (w2[r]) ((float *)r2)[i2[r]] = sum2[r];
    } else {
      if (w1[r]) ((uint16_t *)r1)[i1[r]] = (uint16_t)bf16_bits_rtne(sum1[r]);
      if (w2[r]) ((uint16_t *)r2)[i2[r]] = (uint16_t)bf16_bits_rtne(sum2[r]);
    }
  }
}

// ---------------------------------------------------------------------------------------------------------------
template <bool TABLE_F32>
__device__ __forceinline__ float table_at(const void *table, int64_t off) {
  if constexpr (TABLE_F32) return ((const float *)table)[off];
  else return bf16_bits_to_f32(((const uint16_t *)table)[off]);
}

template <bool TABLE_F32, int CPL>
__global__ void __launch_bounds__(kTrainThreads)
    bag_backward_kernel(const float *__restrict__ grad_out, const int64_t *__restrict__ idx,
                        const float *__restrict__ w, int K, const void *__restrict__ table, int64_t rows, int D,
                        float *__restrict__ acc, uint8_t *__restrict__ touched, float *__restrict__ gw) {
  const int64_t n = blockIdx.x;
  const int wave = threadIdx.x / kWave, lane = lane_id();
  float g[CPL];
#pragma unroll
  for (int e = 0; e < CPL; ++e) {
    const int d = lane + kWave * e;
    g[e] = d < D ? grad_out[n * D + d] : 0.f;
  }
  for (int k0 = wave * kBagInFlight; k0 < K; k0 += kTrainWaves * kBagInFlight) {
    int64_t r[kBagInFlight];
    float wk[kBagInFlight], t[kBagInFlight][CPL];
    bool ok[kBagInFlight];
#pragma unroll
    for (int u = 0; u < kBagInFlight; ++u) {
      const int k = k0 + u;
      const bool live = k < K;                         // wavefront-uniform
      const int64_t rr = live ? idx[n * K + k] : 0;
      ok[u] = live && rr >= 0 && rr < rows;
      r[u] = ok[u] ? rr : 0;
      wk[u] = live ? w[n * K + k] : 0.f;
#pragma unroll
      for (int e = 0; e < CPL; ++e) {
        const int d = lane + kWave * e;
        t[u][e] = d < D ? table_at<TABLE_F32>(table, r[u] * D + d) : 0.f;
      }
    }
#pragma unroll
    for (int u = 0; u < kBagInFlight; ++u) {
      const int k = k0 + u;
      if (k >= K) continue;
      float dot = 0.f;
#pragma unroll
      for (int e = 0; e < CPL; ++e) dot = fmaf(g[e], t[u][e], dot);
      dot = wave_sum_f32(dot);
      if (lane == 0) gw[n * K + k] = ok[u] ? dot : __builtin_nanf("");  // an index outside the table: NaN
      if (!ok[u]) continue;
#pragma unroll
      for (int e = 0; e < CPL; ++e) {
        const int d = lane + kWave * e;
        if (d < D) unsafeAtomicAdd(acc + r[u] * D + d, wk[u] * g[e]);
      }
      if (lane == 0) touched[r[u]] = 1;
    }
  }
}

// ---------------------------------------------------------------------------------------------------------------
// The bag backward with the lookups of a few tokens grouped by table row first: 512 lookups per workgroup (T = 512
// / K tokens, fewer where T x D gradients exceed the LDS stage), sorted in the workgroup by (row, lookup) with a
// bitonic network over its 512 threads (distances below 64 by lane exchange, the rest through LDS).  Each
// wavefront then owns 64 consecutive sorted lookups and walks the runs of equal rows among them: one table-row read
// per run, the run's sum of w x g in registers and ONE set of atomic adds per run, so a row read by many tokens
// (Zipf-skewed indices) costs one atomic per run instead of one per lookup.  Runs keep the lookups' order, so
// the in-register sum adds the products in lookup order.
constexpr int kSortEntries = 512;
constexpr int kSortThreads = kSortEntries;  // one key per thread
constexpr int kSortShift = 9;               // key = row << 9 | lookup slot
constexpr int kStageFloats = 4096;          // LDS for the T x D staged token gradients (16 KB)
constexpr int kRunsInFlight = 4;            // runs per wavefront whose table-row loads are issued together
constexpr uint64_t kNoKey = ~0ull;          // padding and lookups outside the table sort last

// one compare-exchange of an ascending bitonic sort over the workgroup's threads (block K, distance J)
template <int K, int J>
__device__ __forceinline__ uint64_t sort_step(uint64_t key, uint64_t *sKey, int t) {
  uint64_t other;
  if constexpr (J >= kWave) {
    sKey[t] = key;
    __syncthreads();
    other = sKey[t ^ J];
    __syncthreads();
  } else {
    other = xor_lane64<J>(key);
  }
  const bool keep_min = ((t & J) == 0) == ((t & K) == 0);
  const uint64_t lo = key < other ? key : other, hi = key < other ? other : key;
  return keep_min ? lo : hi;
}

template <int K, int J>
__device__ __forceinline__ uint64_t sort_merge(uint64_t key, uint64_t *sKey, int t) {
  key = sort_step<K, J>(key, sKey, t);
  if constexpr (J > 1) return sort_merge<K, J / 2>(key, sKey, t);
  else return key;
}

template <int K>
__device__ __forceinline__ uint64_t sort_keys(uint64_t key, uint64_t *sKey, int t) {
  key = sort_merge<K, K / 2>(key, sKey, t);
  if constexpr (K < kSortEntries) return sort_keys<K * 2>(key, sKey, t);
  else return key;
}

__device__ __forceinline__ int64_t readlane64(int64_t v, int l) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, l);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)((uint64_t)v >> 32), l);
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

template <bool TABLE_F32, int CPL>
__global__ void __launch_bounds__(kSortThreads)
    bag_backward_sorted_kernel(const float *__restrict__ grad_out, const int64_t *__restrict__ idx,
                               const float *__restrict__ w, int64_t N, int K, int T,
                               const void *__restrict__ table, int64_t rows, int D, float *__restrict__ acc,
                               uint8_t *__restrict__ touched, float *__restrict__ gw) {
  __shared__ float sG[kStageFloats];
  __shared__ uint64_t sKey[kSortEntries];
  __shared__ float sW[kSortEntries], sGW[kSortEntries];
  const int t = threadIdx.x, lane = lane_id();
  const int64_t n0 = (int64_t)blockIdx.x * T;
  const int nT = (int)(N - n0 < T ? N - n0 : T);
  const int E = nT * K;                       // <= 512
  const int64_t e0 = n0 * K;
  for (int i = t; i < nT * D; i += kSortThreads) sG[i] = grad_out[n0 * D + i];
  uint64_t key = kNoKey;
  if (t < E) {
    const int64_t r = idx[e0 + t];
    sW[t] = w[e0 + t];
    if (r >= 0 && r < rows) key = ((uint64_t)r << kSortShift) | (uint64_t)t;
    else sGW[t] = __builtin_nanf("");         // an index outside the table: NaN weight gradient, no update
  }
  key = sort_keys<2>(key, sKey, t);
  __syncthreads();                            // staged gradients and weights visible to every wavefront

  const bool valid = key != kNoKey;
  const int64_t row = (int64_t)(key >> kSortShift);
  const int slot = (int)(key & (kSortEntries - 1));
  // the previous lane's row (lane 0 starts a run by definition)
  const uint32_t plo = (uint32_t)__shfl_up((int)(uint32_t)row, 1, kWave);
  const uint32_t phi = (uint32_t)__shfl_up((int)(uint32_t)((uint64_t)row >> 32), 1, kWave);
  const int64_t prow = (int64_t)(((uint64_t)phi << 32) | plo);
  uint64_t heads = ballot(valid && (lane == 0 || prow != row));
  const int nvalid = __popcll(ballot(valid));  // valid keys precede the padding
  const int my_n = valid ? slot / K : 0;
  const float my_w = valid ? sW[slot] : 0.f;

  while (heads) {
    int h[kRunsInFlight], end[kRunsInFlight];
    int64_t r[kRunsInFlight];
    float tv[kRunsInFlight][CPL];
#pragma unroll
    for (int u = 0; u < kRunsInFlight; ++u) {
      h[u] = heads ? __builtin_ctzll(heads) : kWave;
      heads = heads ? heads & (heads - 1) : 0;
    }
#pragma unroll
    for (int u = 0; u < kRunsInFlight; ++u) {
      const int nxt = u + 1 < kRunsInFlight ? h[u + 1] : (heads ? __builtin_ctzll(heads) : kWave);
      end[u] = nxt < kWave ? nxt : nvalid;
      r[u] = h[u] < kWave ? readlane64(row, h[u]) : 0;
#pragma unroll
      for (int e = 0; e < CPL; ++e) {
        const int d = lane + kWave * e;
        tv[u][e] = (h[u] < kWave && d < D) ? table_at<TABLE_F32>(table, r[u] * D + d) : 0.f;
      }
    }
#pragma unroll
    for (int u = 0; u < kRunsInFlight; ++u) {
      if (h[u] >= kWave) break;               // wavefront-uniform
      float s[CPL];
#pragma unroll
      for (int e = 0; e < CPL; ++e) s[e] = 0.f;
      for (int j = h[u]; j < end[u]; ++j) {
        const int nj = __builtin_amdgcn_readlane(my_n, j);
        const float wj = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, my_w), j));
        const float *g = sG + nj * D;
        float dot = 0.f;
#pragma unroll
        for (int e = 0; e < CPL; ++e) {
          const int d = lane + kWave * e;
          const float gv = d < D ? g[d] : 0.f;
          dot = fmaf(gv, tv[u][e], dot);
          s[e] = s[e] + wj * gv;
        }
        dot = wave_sum_f32(dot);
        if (lane == 0) sGW[__builtin_amdgcn_readlane(slot, j)] = dot;
      }
#pragma unroll
      for (int e = 0; e < CPL; ++e) {
        const int d = lane + kWave * e;
        if (d < D) unsafeAtomicAdd(acc + r[u] * D + d, s[e]);
      }
      if (lane == 0) touched[r[u]] = 1;
    }
  }
  __syncthreads();
  for (int i = t; i < E; i += kSortThreads) gw[e0 + i] = sGW[i];
}

// ---------------------------------------------------------------------------------------------------------------
// state: 0 fp32 moments, 1 bf16 moments, 2 int8 / uint8 codes + fp32 row scales.  Column layout of a row in its
// wavefront: chunk c, lane l, element i holds column c * 64 * V + l * V + i.  V = 4 (D a multiple of 4) gives each
// lane 16-byte fp32, 8-byte bf16 and 4-byte int8 accesses; V = 2 (256 < D <= 384: 3 chunks, no idle slots at
// D = 384) 8-, 4- and 2-byte accesses; V = 1 is the fallback for other widths.
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

template <int V>
__device__ __forceinline__ void load_f32v(const float *q, bool in, float *x) {
  if constexpr (V == 4) {
    const f32x4 t = in ? *(const f32x4 *)q : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = t[i];
  } else if constexpr (V == 2) {
    const f32x2 t = in ? *(const f32x2 *)q : f32x2{0.f, 0.f};
    x[0] = t[0];
    x[1] = t[1];
  } else {
    x[0] = in ? *q : 0.f;
  }
}
template <int V>
__device__ __forceinline__ void store_f32v(float *q, const float *x) {
  if constexpr (V == 4) *(f32x4 *)q = f32x4{x[0], x[1], x[2], x[3]};
  else if constexpr (V == 2) *(f32x2 *)q = f32x2{x[0], x[1]};
  else *q = x[0];
}
template <int V>
__device__ __forceinline__ void load_bf16v(const uint16_t *q, bool in, float *x) {
  if constexpr (V == 4) {
    const u32x2 t = in ? *(const u32x2 *)q : u32x2{0u, 0u};
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = bf16_bits_to_f32((t[i / 2] >> (16 * (i % 2))) & 0xFFFFu);
  } else if constexpr (V == 2) {
    const uint32_t t = in ? *(const uint32_t *)q : 0u;
    x[0] = bf16_bits_to_f32(t & 0xFFFFu);
    x[1] = bf16_bits_to_f32(t >> 16);
  } else {
    x[0] = in ? bf16_bits_to_f32(*q) : 0.f;
  }
}
template <int V>
__device__ __forceinline__ void store_bf16v(uint16_t *q, const float *x) {
  if constexpr (V == 4) {
    *(u32x2 *)q = u32x2{bf16_bits_rtne(x[0]) | (bf16_bits_rtne(x[1]) << 16),
                        bf16_bits_rtne(x[2]) | (bf16_bits_rtne(x[3]) << 16)};
  } else if constexpr (V == 2) {
    *(uint32_t *)q = bf16_bits_rtne(x[0]) | (bf16_bits_rtne(x[1]) << 16);
  } else {
    *q = (uint16_t)bf16_bits_rtne(x[0]);
  }
}
// int8 first-moment codes (signed) or uint8 second-moment codes, as floats
template <int V, bool SIGNED>
__device__ __forceinline__ void load_codes(const uint8_t *q, bool in, float *x) {
  if constexpr (V == 4) {
    const uint32_t t = in ? *(const uint32_t *)q : 0u;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t c = (t >> (8 * i)) & 0xFFu;
      x[i] = SIGNED ? (float)(int8_t)c : (float)c;
    }
  } else if constexpr (V == 2) {
    const uint32_t t = in ? *(const uint16_t *)q : 0u;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const uint32_t c = (t >> (8 * i)) & 0xFFu;
      x[i] = SIGNED ? (float)(int8_t)c : (float)c;
    }
  } else {
    x[0] = !in ? 0.f : SIGNED ? (float)*(const int8_t *)q : (float)*q;
  }
}
template <int V>
__device__ __forceinline__ void store_codes(uint8_t *q, const float *x) {
  if constexpr (V == 4) {
    uint32_t t = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) t |= ((uint32_t)(int)x[i] & 0xFFu) << (8 * i);
    *(uint32_t *)q = t;
  } else if constexpr (V == 2) {
    *(uint16_t *)q = (uint16_t)((((uint32_t)(int)x[0]) & 0xFFu) | ((((uint32_t)(int)x[1]) & 0xFFu) << 8));
  } else {
    *q = (uint8_t)(int)x[0];
  }
}

// c / DEN rounded to nearest for an integer code c (|c| <= 127 for DEN 127, 0 <= c <= 255 for DEN 255): the product
// with the rounded reciprocal, corrected once by its fma residual.  Equal to the IEEE quotient for every such code
// (checked exhaustively in exact arithmetic), at 3 instructions instead of the 10 of a general division.
template <int DEN>
__device__ __forceinline__ float div_code(float c) {
  constexpr float r = 1.0f / DEN;
  const float q = c * r;
  const float e = __builtin_fmaf(-q, (float)DEN, c);
  return __builtin_fmaf(e, r, q);
}

template <int STATE, int V, int NC>
__global__ void __launch_bounds__(kTrainThreads)
    lazy_adam_kernel(float *__restrict__ p, void *__restrict__ m_ptr, void *__restrict__ v_ptr,
                     float *__restrict__ m_scale, float *__restrict__ v_scale, float *__restrict__ acc,
                     uint8_t *__restrict__ touched, const float *__restrict__ grad_scale, int64_t rows, int D,
                     float step_size, float bc2_sqrt, float beta1, float beta2, float omb1, float omb2, float eps) {
  constexpr int L = V * NC;                   // columns per lane
  const int lane = lane_id();
  const float scale = *grad_scale;
  for (int64_t row = (int64_t)blockIdx.x * kTrainWaves + threadIdx.x / kWave; row < rows;
       row += (int64_t)gridDim.x * kTrainWaves) {
    if (touched[row] == 0) continue;                   // wavefront-uniform: one wavefront per row
    float g[L], m[L], v[L], pv[L];
    bool in[NC];
    int64_t off[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int d0 = c * kWave * V + lane * V;
      in[c] = d0 < D;                                  // D % V == 0: all V columns in or all out
      off[c] = row * D + (in[c] ? d0 : 0);
      load_f32v<V>(acc + off[c], in[c], g + c * V);
      load_f32v<V>(p + off[c], in[c], pv + c * V);
      if constexpr (STATE == 0) {
        load_f32v<V>((const float *)m_ptr + off[c], in[c], m + c * V);
        load_f32v<V>((const float *)v_ptr + off[c], in[c], v + c * V);
      } else if constexpr (STATE == 1) {
        load_bf16v<V>((const uint16_t *)m_ptr + off[c], in[c], m + c * V);
        load_bf16v<V>((const uint16_t *)v_ptr + off[c], in[c], v + c * V);
      } else {
        load_codes<V, true>((const uint8_t *)m_ptr + off[c], in[c], m + c * V);
        load_codes<V, false>((const uint8_t *)v_ptr + off[c], in[c], v + c * V);
      }
    }
#pragma unroll
    for (int e = 0; e < L; ++e) g[e] = g[e] * scale;
    if constexpr (STATE == 2) {  // decode: m = sign * (c / 127)^2 * scale, v = ((c / 255) * scale)^4
      const float ms = m_scale[row], vs = v_scale[row];
#pragma unroll
      for (int e = 0; e < L; ++e) {
        float mm = div_code<127>(m[e]);
        mm = (mm < 0.f ? -1.0f : 1.0f) * mm * mm * ms;
        float vv = div_code<255>(v[e]) * vs;
        vv = vv * vv;
        vv = vv * vv;
        m[e] = mm;
        v[e] = vv;
      }
    }
    float mq[L], vroot[L];
    float mmax = 0.f, vmax = 0.f;
#pragma unroll
    for (int e = 0; e < L; ++e) {
      if constexpr (STATE == 0) {  // the fp32 kernel forms 1 - beta on the device
        m[e] = beta1 * m[e] + (1.0f - beta1) * g[e];
        v[e] = beta2 * v[e] + (1.0f - beta2) * g[e] * g[e];
        pv[e] = pv[e] - step_size * m[e] / (sqrtf(v[e]) / bc2_sqrt + eps);
      } else {
        m[e] = beta1 * m[e] + omb1 * g[e];
        v[e] = beta2 * v[e] + omb2 * g[e] * g[e];
        const float denom = sqrtf(v[e]) / bc2_sqrt + eps;
        pv[e] = pv[e] - (step_size * m[e]) / denom;
      }
      if constexpr (STATE == 2) {
        vroot[e] = sqrtf(sqrtf(v[e]));
        if (in[e / V]) {
          mmax = fmaxf(mmax, fabsf(m[e]));
          vmax = fmaxf(vmax, vroot[e]);
        }
      }
    }
    if constexpr (STATE == 2) {  // encode against the row's largest |m| and v^(1/4)
      mmax = wave_max_f32(mmax);
      vmax = wave_max_f32(vmax);
      const float md = mmax > 0.f ? mmax : 1.0f, vd = vmax > 0.f ? vmax : 1.0f;
#pragma unroll
      for (int e = 0; e < L; ++e) {
        float a = sqrtf(fabsf(m[e]) / md);
        a = (m[e] < 0.f ? -1.0f : 1.0f) * a * 127.0f;
        float b = vroot[e] / vd * 255.0f;
        a = rintf(fminf(fmaxf(a, -127.0f), 127.0f));
        b = rintf(fminf(fmaxf(b, 0.0f), 255.0f));
        b = v[e] > 0.f ? fmaxf(b, 1.0f) : 0.0f;  // a positive second moment never gets a zero code
        mq[e] = a;
        vroot[e] = b;
      }
      if (lane == 0) {
        m_scale[row] = mmax;
        v_scale[row] = vmax;
      }
    }
    const float zero[V] = {};
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      if (!in[c]) continue;
      store_f32v<V>(p + off[c], pv + c * V);
      store_f32v<V>(acc + off[c], zero);
      if constexpr (STATE == 0) {
        store_f32v<V>((float *)m_ptr + off[c], m + c * V);
        store_f32v<V>((float *)v_ptr + off[c], v + c * V);
      } else if constexpr (STATE == 1) {
        store_bf16v<V>((uint16_t *)m_ptr + off[c], m + c * V);
        store_bf16v<V>((uint16_t *)v_ptr + off[c], v + c * V);
      } else {
        store_codes<V>((uint8_t *)m_ptr + off[c], mq + c * V);
        store_codes<V>((uint8_t *)v_ptr + off[c], vroot + c * V);
      }
    }
    if (lane == 0) touched[row] = 0;
  }
}

// The bag backward without the per-sample-weight gradient (its caller discards it when the weights do not train: the
// unit weights of the Engram lookups, smlm/engram.py:118): acc[idx[i]] += w[i] * g[i / K] (w[i] = 1 when w is null)
// and touched[idx[i]] = 1 for the L = N * K lookups i, in no fixed order (fp32 atomic adds), with no table read and
// no sort.  One thread per element, so the lanes of an atomic instruction cover contiguous columns of 64 / D rows
// (Engram: 24-column rows, 2.7 rows per instruction).  Timing probe at the Engram shape (262,144 lookups of 24 into
// 8.4M rows): 31 us this way, 109 us with 16 bytes per lane (each instruction then spreads its lanes over 10 rows at
// a 16-byte stride, and four instructions revisit each row).  WIDE: 64-bit element indices.  An index outside
// [0, rows) adds nothing.
template <bool WIDE>
__global__ void __launch_bounds__(kTrainThreads)
    row_scatter_kernel(const float *__restrict__ g, const int64_t *__restrict__ idx, const float *__restrict__ w,
                       int64_t L, int K, int D, int64_t rows, float *__restrict__ acc, uint8_t *__restrict__ touched) {
  typedef typename std::conditional<WIDE, uint64_t, uint32_t>::type index_t;
  const index_t total = (index_t)(L * D), stride = (index_t)gridDim.x * kTrainThreads;
  for (index_t t = (index_t)blockIdx.x * kTrainThreads + threadIdx.x; t < total; t += stride) {
    const index_t i = t / (index_t)D;
    const int d = (int)(t - i * (index_t)D);
    const int64_t r = idx[i];
    if (r < 0 || r >= rows) continue;
    const float v = g[(int64_t)(K == 1 ? i : i / (index_t)K) * D + d];
    unsafeAtomicAdd(acc + r * D + d, w ? w[i] * v : v);
    if (d == 0) touched[r] = 1;
  }
}

void launch_row_scatter(const float *g, const int64_t *idx, const float *w, int64_t L, int K, int D, int64_t rows,
                        float *acc, uint8_t *touched, hipStream_t stream) {
  const int64_t total = L * D;
  const dim3 grid((unsigned)std::min<int64_t>((total + kTrainThreads - 1) / kTrainThreads, 1 << 20)),
      block(kTrainThreads);
  if (total + (int64_t)grid.x * kTrainThreads <= (int64_t)UINT32_MAX)  // t + stride stays within 32 bits
    hipLaunchKernelGGL((row_scatter_kernel<false>), grid, block, 0, stream, g, idx, w, L, K, D, rows, acc, touched);
  else
    hipLaunchKernelGGL((row_scatter_kernel<true>), grid, block, 0, stream, g, idx, w, L, K, D, rows, acc, touched);
}

template <int CPL>
void launch_bag_backward(const float *grad_out, const int64_t *idx, const float *w, int64_t N, int K,
                         const void *table, bool f32, int64_t rows, int D, float *acc, uint8_t *touched, float *gw,
                         hipStream_t stream) {
  if (K <= kSortEntries) {  // T tokens per workgroup: T x K <= 512 lookups, T x D <= 4096 staged floats
    const int T = std::min(kSortEntries / K, kStageFloats / D);
    const dim3 grid((unsigned)((N + T - 1) / T)), block(kSortThreads);
    if (f32)
      hipLaunchKernelGGL((bag_backward_sorted_kernel<true, CPL>), grid, block, 0, stream, grad_out, idx, w, N, K, T,
                         table, rows, D, acc, touched, gw);
    else
      hipLaunchKernelGGL((bag_backward_sorted_kernel<false, CPL>), grid, block, 0, stream, grad_out, idx, w, N, K,
                         T, table, rows, D, acc, touched, gw);
    return;
  }
  if (f32)
    hipLaunchKernelGGL((bag_backward_kernel<true, CPL>), dim3((unsigned)N), dim3(kTrainThreads), 0, stream, grad_out,
                       idx, w, K, table, rows, D, acc, touched, gw);
  else
    hipLaunchKernelGGL((bag_backward_kernel<false, CPL>), dim3((unsigned)N), dim3(kTrainThreads), 0, stream,
                       grad_out, idx, w, K, table, rows, D, acc, touched, gw);
}

bool aligned(const void *p, int a) { return ((uintptr_t)p % a) == 0; }

template <int STATE>
void launch_adam(float *p, void *m, void *v, float *ms, float *vs, float *acc, uint8_t *touched,
                 const float *grad_scale, int64_t rows, int D, float step_size, float bc2_sqrt, float b1, float b2,
                 float omb1, float omb2, float eps, hipStream_t stream) {
  int64_t blocks = (rows + kTrainWaves - 1) / kTrainWaves;
  // one row per wavefront up to 1,048,576 rows, grid-stride beyond (B-1M, all rows touched: fp32 2.53 -> 2.43 ms,
  // bf16 1.91 -> 1.78, int8 1.62 -> 1.52 against 4 rows per wavefront; 16 rows per wavefront 2.59 / 1.95 / 1.62)
  if (blocks > (1 << 18)) blocks = 1 << 18;
  const dim3 grid((unsigned)blocks), block(kTrainThreads);
  constexpr int kMomentBytes = STATE == 0 ? 4 : STATE == 1 ? 2 : 1;
  const bool vec = D % 4 == 0 && aligned(p, 16) && aligned(acc, 16) && aligned(m, 4 * kMomentBytes) &&
                   aligned(v, 4 * kMomentBytes);
#define SMLM_ADAM(V, NC)                                                                                       \
  hipLaunchKernelGGL((lazy_adam_kernel<STATE, V, NC>), grid, block, 0, stream, p, m, v, ms, vs, acc, touched,   \
                     grad_scale, rows, D, step_size, bc2_sqrt, b1, b2, omb1, omb2, eps)
  if (vec && D <= 256) SMLM_ADAM(4, 1);
  else if (vec && D <= 384) SMLM_ADAM(2, 3);
  else if (vec) SMLM_ADAM(4, 2);
  else if (D <= 128) SMLM_ADAM(1, 2);
  else if (D <= 256) SMLM_ADAM(1, 4);
  else if (D <= 384) SMLM_ADAM(1, 6);
  else SMLM_ADAM(1, 8);
#undef SMLM_ADAM
}


}  // namespace
}  // namespace smlm

extern "C" int smlm_pkm_select_backward(const int64_t *idx, const float *w, const void *g_scores, const float *g_w,
                                        int dtype, int64_t N, int H, int NK, int knn, void *ds1, void *ds2,
                                        void *stream) {
  using namespace smlm;
  if (!idx || !w || !ds1 || !ds2) return fail(SMLM_EINVAL, "smlm_pkm_select_backward: null idx, w, ds1 or ds2");
  if (dtype != SMLM_BF16 && dtype != SMLM_F32)
    return fail(SMLM_EINVAL, "smlm_pkm_select_backward: dtype must be SMLM_BF16 or SMLM_F32, got %d", dtype);
  if (N < 0 || H < 1 || knn < 1 || knn > 2 * kWave || NK < knn || NK > 65536)
    return fail(SMLM_EUNSUPPORTED, "smlm_pkm_select_backward: N=%lld H=%d NK=%d knn=%d (knn in [1, 128], NK in "
                "[knn, 65536])", (long long)N, H, NK, knn);
  if (!aligned(ds1, 16) || !aligned(ds2, 16))
    return fail(SMLM_EINVAL, "smlm_pkm_select_backward: ds1 and ds2 must be 16-byte aligned");
  const int64_t rows = N * H;
  if (rows == 0) return SMLM_OK;
  const dim3 grid((unsigned)((rows + kTrainWaves - 1) / kTrainWaves)), block(kTrainThreads);
  if (dtype == SMLM_F32)
    hipLaunchKernelGGL((select_backward_kernel<true>), grid, block, 0, (hipStream_t)stream, idx, w, g_scores, g_w,
                       rows, NK, knn, ds1, ds2);
  else
    hipLaunchKernelGGL((select_backward_kernel<false>), grid, block, 0, (hipStream_t)stream, idx, w, g_scores, g_w,
                       rows, NK, knn, ds1, ds2);
  return launch_status("smlm_pkm_select_backward");
}

extern "C" int smlm_bag_backward_rows(const float *grad_out, const int64_t *idx, const float *w, int64_t N, int K,
                                      const void *table, int table_dtype, int64_t rows, int D, float *acc,
                                      uint8_t *touched, float *gw, void *stream) {
  using namespace smlm;
  if (!grad_out || !idx || !acc || !touched || (gw && (!w || !table)))
    return fail(SMLM_EINVAL, "smlm_bag_backward_rows: null pointer argument (w and table are needed with gw)");
  if (!gw) {  // no per-sample-weight gradient: scatter the lookups, no table read
    if (N < 0 || K < 1 || rows < 1 || D < 1 || D > kMaxD || (N > 0 && K > INT64_MAX / D / N))
      return fail(SMLM_EUNSUPPORTED, "smlm_bag_backward_rows: N=%lld K=%d rows=%lld D=%d (1 <= D <= %d)",
                  (long long)N, K, (long long)rows, D, kMaxD);
    if (N == 0) return SMLM_OK;
    launch_row_scatter(grad_out, idx, w, N * K, K, D, rows, acc, touched, (hipStream_t)stream);
    return launch_status("smlm_bag_backward_rows");
  }
  if (table_dtype != SMLM_F32 && table_dtype != SMLM_BF16)
    return fail(SMLM_EINVAL, "smlm_bag_backward_rows: the table must be SMLM_F32 or SMLM_BF16, got %d", table_dtype);
  if (N < 0 || N > 0x7FFFFFFFLL || K < 1 || rows < 1 || rows >= (1LL << (63 - kSortShift)) || D < 1 || D > kMaxD)
    return fail(SMLM_EUNSUPPORTED, "smlm_bag_backward_rows: N=%lld K=%d rows=%lld D=%d (1 <= D <= %d)",
                (long long)N, K, (long long)rows, D, kMaxD);
  if (N == 0) return SMLM_OK;
  const bool f32 = table_dtype == SMLM_F32;
  hipStream_t s = (hipStream_t)stream;
  if (D <= 128) launch_bag_backward<2>(grad_out, idx, w, N, K, table, f32, rows, D, acc, touched, gw, s);
  else if (D <= 256) launch_bag_backward<4>(grad_out, idx, w, N, K, table, f32, rows, D, acc, touched, gw, s);
  else if (D <= 384) launch_bag_backward<6>(grad_out, idx, w, N, K, table, f32, rows, D, acc, touched, gw, s);
  else launch_bag_backward<8>(grad_out, idx, w, N, K, table, f32, rows, D, acc, touched, gw, s);
  return launch_status("smlm_bag_backward_rows");
}

extern "C" int smlm_lazy_adam(float *param, void *exp_avg, void *exp_avg_sq, float *exp_avg_scale,
                              float *exp_avg_sq_scale, int state, float *acc, uint8_t *touched,
                              const float *grad_scale, int64_t rows, int D, float step_size, float bc2_sqrt,
                              float beta1, float beta2, float one_minus_beta1, float one_minus_beta2, float eps,
                              void *stream) {
  using namespace smlm;
  if (!param || !exp_avg || !exp_avg_sq || !acc || !touched || !grad_scale)
    return fail(SMLM_EINVAL, "smlm_lazy_adam: null pointer argument");
  if (state != SMLM_ADAM_F32 && state != SMLM_ADAM_BF16 && state != SMLM_ADAM_INT8)
    return fail(SMLM_EINVAL, "smlm_lazy_adam: unknown moment storage %d", state);
  if (state == SMLM_ADAM_INT8 && (!exp_avg_scale || !exp_avg_sq_scale))
    return fail(SMLM_EINVAL, "smlm_lazy_adam: int8 moments need exp_avg_scale and exp_avg_sq_scale");
  if (rows < 0 || D < 1 || D > kMaxD)
    return fail(SMLM_EUNSUPPORTED, "smlm_lazy_adam: rows=%lld D=%d (1 <= D <= %d)", (long long)rows, D, kMaxD);
  if (rows == 0) return SMLM_OK;
  hipStream_t s = (hipStream_t)stream;
  if (state == SMLM_ADAM_F32)
    launch_adam<0>(param, exp_avg, exp_avg_sq, exp_avg_scale, exp_avg_sq_scale, acc, touched, grad_scale, rows, D,
                   step_size, bc2_sqrt, beta1, beta2, one_minus_beta1, one_minus_beta2, eps, s);
  else if (state == SMLM_ADAM_BF16)
    launch_adam<1>(param, exp_avg, exp_avg_sq, exp_avg_scale, exp_avg_sq_scale, acc, touched, grad_scale, rows, D,
                   step_size, bc2_sqrt, beta1, beta2, one_minus_beta1, one_minus_beta2, eps, s);
  else
    launch_adam<2>(param, exp_avg, exp_avg_sq, exp_avg_scale, exp_avg_sq_scale, acc, touched, grad_scale, rows, D,
                   step_size, bc2_sqrt, beta1, beta2, one_minus_beta1, one_minus_beta2, eps, s);
  return launch_status("smlm_lazy_adam");
}
