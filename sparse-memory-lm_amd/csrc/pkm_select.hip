// Product-key selection (kernels 2 and 3): per (token, head) the top-knn of both sub-key score rows, the
// top-knn of the (i+1)(j+1) <= knn Cartesian candidates and the fp32 softmax.  Replaces pk_select /
// _pk_select_kernel (smlm/kernels.py:128-177, 200-226) with the same deterministic semantics, and extends them
// to fp32 scores (smlm/pkm.py:125-136 for the fp32 path):
//   - a half's element k gets the key (order(score) << kIdxBits) | (idxmax - k): larger key = larger score,
//     ties -> smaller k.  bf16: 16-bit code + 16-bit index in a u32; fp32: 32 + 32 bits in a u64.
//   - candidate (i, j) is scored as dtype(v1[i] + v2[j]) (bf16: fp32 add, rounded to nearest even) with key
//     (order(score) << 32) | (0xFFFFFFFF - (i1*NK + i2)), so ties -> smaller table index.
//   - all keys are distinct, so "the knn largest keys" is one exact set.
//
// One workgroup = two wavefronts per (token, head) row; wavefront 0 selects in s1, wavefront 1 in s2, then
// wavefront 0 does the Cartesian step.  A wavefront's half top-k:
//   1. every lane takes the maximum key of its strided share of the row; the knn-th largest of the 64 lane
//      maxima is a threshold t0 that at least knn elements reach (the knn largest lane maxima are distinct
//      elements), found by a bitwise search over ballot() counts;
//   2. the elements >= t0 (typically a few dozen) are compacted into LDS with ballot/mbcnt;
//   3. the exact knn-th largest key t1 among them is found by the same bitwise search, the knn keys >= t1 are
//      compacted and put in descending order by counting ranks.
// If more than kCap elements reach t0 (adversarial rows), step 3 runs directly on the row instead.
#include "pkm_common.h"

namespace smlm {
namespace {

constexpr int kCap = 1024;       // LDS candidates per half
constexpr int kMaxKnn = 64;
constexpr int kMaxPairs = 288;   // (i, j) with (i+1)(j+1) <= 64: sum_{i=1..64} floor(64/i) = 280

template <bool F32> struct SelKey;
template <> struct SelKey<false> { using T = uint32_t; };
template <> struct SelKey<true> { using T = uint64_t; };

template <bool F32>
__device__ __forceinline__ typename SelKey<F32>::T half_key(const void *row, int k) {
  if constexpr (F32) {
    const uint32_t u = ((const uint32_t *)row)[k];
    return ((uint64_t)order32(u) << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)k);
  } else {
    const uint32_t b = ((const uint16_t *)row)[k];
    return (order16(b) << 16) | (0xFFFFu - (uint32_t)k);
  }
}
template <bool F32>
__device__ __forceinline__ float key_value(typename SelKey<F32>::T key) {
  if constexpr (F32) return __uint_as_float(unorder32((uint32_t)(key >> 32)));
  else return bf16_bits_to_f32(unorder16(key >> 16));
}
template <bool F32>
__device__ __forceinline__ uint32_t key_index(typename SelKey<F32>::T key) {
  if constexpr (F32) return 0xFFFFFFFFu - (uint32_t)key;
  else return 0xFFFFu - (key & 0xFFFFu);
}

// Largest t with count_ge(t) >= need (count_ge is wave-uniform and non-increasing in t; count_ge(0) >= need).
template <typename Key, typename CountGE>
__device__ __forceinline__ Key threshold_search(int need, CountGE count_ge) {
  Key t = 0;
  for (int b = (int)sizeof(Key) * 8 - 1; b >= 0; --b) {
    const Key c = t | ((Key)1 << b);
    if (count_ge(c) >= need) t = c;
  }
  return t;
}

// Exact top-knn keys of one score row (NK elements), written to out[0..knn) in descending order.
template <bool F32>
__device__ void half_topk(const void *row, int NK, int knn, typename SelKey<F32>::T *cand,
                          typename SelKey<F32>::T *sel, typename SelKey<F32>::T *out) {
  using Key = typename SelKey<F32>::T;
  const int lane = lane_id();

  Key mx = 0;
  for (int k = lane; k < NK; k += kWave) {
    const Key u = half_key<F32>(row, k);
    mx = u > mx ? u : mx;
  }
  const Key t0 = threshold_search<Key>(knn, [&](Key t) { return (int)__popcll(ballot(mx >= t)); });

  int C = 0;
  for (int k0 = 0; k0 < NK; k0 += kWave) {
    const int k = k0 + lane;
    const Key u = k < NK ? half_key<F32>(row, k) : (Key)0;
    const bool take = k < NK && u >= t0;
    const uint64_t m = ballot(take);
    const int pos = C + lanes_below(m);
    if (take && pos < kCap) cand[pos] = u;
    C += (int)__popcll(m);
  }
  wave_lds_sync();

  const bool in_lds = C <= kCap;
  Key t1;
  if (in_lds) {
    t1 = threshold_search<Key>(knn, [&](Key t) {
      int cnt = 0;
      for (int p0 = 0; p0 < C; p0 += kWave) {
        const int p = p0 + lane;
        cnt += (int)__popcll(ballot(p < C && cand[p] >= t));
      }
      return cnt;
    });
  } else {
    t1 = threshold_search<Key>(knn, [&](Key t) {
      int cnt = 0;
      for (int k0 = 0; k0 < NK; k0 += kWave) {
        const int k = k0 + lane;
        cnt += (int)__popcll(ballot(k < NK && half_key<F32>(row, k) >= t));
      }
      return cnt;
    });
  }

  // exactly knn keys are >= t1
  int S = 0;
  const int total = in_lds ? C : NK;
  for (int p0 = 0; p0 < total; p0 += kWave) {
    const int p = p0 + lane;
    Key u = 0;
    if (p < total) u = in_lds ? cand[p] : half_key<F32>(row, p);
    const bool ge = p < total && u >= t1;
    const uint64_t m = ballot(ge);
    const int pos = S + lanes_below(m);
    if (ge && pos < kMaxKnn) sel[pos] = u;
    S += (int)__popcll(m);
  }
  wave_lds_sync();
  if (lane < knn) {
    const Key u = sel[lane];
    int rank = 0;
    for (int j = 0; j < knn; ++j) rank += sel[j] > u;
    out[rank] = u;
  }
  wave_lds_sync();
}

template <bool F32>
__global__ void __launch_bounds__(128) select_kernel(const void *__restrict__ s1, const void *__restrict__ s2,
                                                     int NK, int knn, void *__restrict__ scores,
                                                     int64_t *__restrict__ idx, float *__restrict__ w) {
  using Key = typename SelKey<F32>::T;
  __shared__ Key s_cand[2][kCap];
  __shared__ Key s_sel[2][kMaxKnn];
  __shared__ Key s_top[2][kMaxKnn];
  __shared__ uint64_t s_ck[kMaxPairs];
  __shared__ uint64_t s_fsel[kMaxKnn];
  __shared__ uint64_t s_fin[kMaxKnn];

  const int wave = threadIdx.x / kWave;
  const int lane = lane_id();
  const int64_t row = blockIdx.x;  // n * H + h
  const size_t esz = F32 ? 4 : 2;
  const void *src = (const char *)(wave == 0 ? s1 : s2) + row * (int64_t)NK * esz;
  half_topk<F32>(src, NK, knn, s_cand[wave], s_sel[wave], s_top[wave]);
  __syncthreads();
  if (wave != 0) return;

  // Cartesian candidates: lane i < knn owns pairs (i, j), j < knn / (i + 1), at offset sum_{i'<i} knn/(i'+1)
  const int cnt = lane < knn ? knn / (lane + 1) : 0;
  int incl = cnt;
  for (int o = 1; o < kWave; o <<= 1) {
    const int v = __shfl_up(incl, o, kWave);
    if (lane >= o) incl += v;
  }
  const int P = __shfl(incl, kWave - 1, kWave);
  const int off = incl - cnt;
  if (lane < knn) {
    const Key k1 = s_top[0][lane];
    const float v1 = key_value<F32>(k1);
    const uint32_t i1 = key_index<F32>(k1);
    for (int j = 0; j < cnt; ++j) {
      const Key k2 = s_top[1][j];
      const float s = v1 + key_value<F32>(k2);
      const uint32_t code = F32 ? order32(__float_as_uint(s)) : order16(bf16_bits_rtne(s));
      const uint32_t full = i1 * (uint32_t)NK + key_index<F32>(k2);
      s_ck[off + j] = ((uint64_t)code << 32) | (uint64_t)(0xFFFFFFFFu - full);
    }
  }
  wave_lds_sync();

  const uint64_t t = threshold_search<uint64_t>(knn, [&](uint64_t c) {
    int n = 0;
    for (int p0 = 0; p0 < P; p0 += kWave) {
      const int p = p0 + lane;
      n += (int)__popcll(ballot(p < P && s_ck[p] >= c));
    }
    return n;
  });
  int S = 0;
  for (int p0 = 0; p0 < P; p0 += kWave) {
    const int p = p0 + lane;
    const uint64_t u = p < P ? s_ck[p] : 0;
    const bool ge = p < P && u >= t;
    const uint64_t m = ballot(ge);
    const int pos = S + lanes_below(m);
    if (ge && pos < kMaxKnn) s_fsel[pos] = u;
    S += (int)__popcll(m);
  }
  wave_lds_sync();
  if (lane < knn) {
    const uint64_t u = s_fsel[lane];
    int rank = 0;
    for (int j = 0; j < knn; ++j) rank += s_fsel[j] > u;
    s_fin[rank] = u;
  }
  wave_lds_sync();

  float sc = 0.f;
  uint32_t full = 0;
  uint32_t code = 0;
  if (lane < knn) {
    const uint64_t u = s_fin[lane];
    code = (uint32_t)(u >> 32);
    full = 0xFFFFFFFFu - (uint32_t)u;
    sc = F32 ? __uint_as_float(unorder32(code)) : bf16_bits_to_f32(unorder16(code));
  }
  const float mxs = __shfl(sc, 0, kWave);  // descending: lane 0 holds the largest score
  const float e = lane < knn ? expf(sc - mxs) : 0.f;
  const float sum = wave_sum(e);
  if (lane < knn) {
    const int64_t o = row * knn + lane;
    if constexpr (F32) ((float *)scores)[o] = sc;
    else ((uint16_t *)scores)[o] = (uint16_t)unorder16(code);
    idx[o] = (int64_t)full;
    w[o] = e / sum;
  }
}

}  // namespace
}  // namespace smlm

extern "C" int smlm_pkm_select(const void *s1, const void *s2, int dtype, int64_t N, int H, int NK, int knn,
                               void *scores, int64_t *idx, float *w, void *stream) {
  using namespace smlm;
  if (!s1 || !s2 || !scores || !idx || !w)
    return fail(SMLM_EINVAL, "smlm_pkm_select: null s1, s2, scores, idx or w pointer");
  if (dtype != SMLM_BF16 && dtype != SMLM_F32)
    return fail(SMLM_EINVAL, "smlm_pkm_select: dtype must be SMLM_BF16 or SMLM_F32, got %d", dtype);
  if (N < 0 || H < 1 || N * (int64_t)H > 0x7FFFFFFFLL)
    return fail(SMLM_EINVAL, "smlm_pkm_select: N=%lld, H=%d out of range", (long long)N, H);
  if (!is_pow2(knn) || knn > kMaxKnn)
    return fail(SMLM_EUNSUPPORTED, "smlm_pkm_select: knn=%d must be a power of two <= %d", knn, kMaxKnn);
  if (!is_pow2(NK) || NK > 65536 || NK < knn)
    return fail(SMLM_EUNSUPPORTED, "smlm_pkm_select: NK=%d must be a power of two in [knn, 65536]", NK);
  if (N == 0) return SMLM_OK;
  const dim3 grid((unsigned)(N * H));
  if (dtype == SMLM_F32)
    hipLaunchKernelGGL(select_kernel<true>, grid, dim3(2 * kWave), 0, (hipStream_t)stream, s1, s2, NK, knn,
                       scores, idx, w);
  else
    hipLaunchKernelGGL(select_kernel<false>, grid, dim3(2 * kWave), 0, (hipStream_t)stream, s1, s2, NK, knn,
                       scores, idx, w);
  return launch_status("smlm_pkm_select");
}
