// Product-key selection (kernels 2 and 3): per (token, head) the top-knn of both sub-key score rows, the
// top-knn of the (i+1)(j+1) <= knn Cartesian candidates and the fp32 softmax.  Replaces pk_select /
// _pk_select_kernel (smlm/kernels.py:128-177, 200-226) with the same deterministic semantics, and extends them
// to fp32 scores (smlm/pkm.py:125-136 for the fp32 path):
//   - a half's element k gets the key (code(score) << B) | (2^B - 1 - k) with code() order-preserving (B = 16
//     for bf16 in a u32, B = 32 for fp32 in a u64): larger key = larger score, ties -> smaller k;
//   - candidate (i, j) is scored as dtype(v1[i] + v2[j]) (bf16: fp32 add, rounded to nearest even) with key
//     (code(score) << 32) | (0xFFFFFFFF - (i1*NK + i2)), so ties -> smaller table index;
//   - all keys are distinct, so "the knn largest keys" is one exact set.
//
// One workgroup = two wavefronts per (token, head) row: wavefront 0 selects in s1, wavefront 1 in s2, then
// wavefront 0 does the Cartesian step (at knn = 32 each sorts half of the pairs and wavefront 0 merges the two).
// Half top-k of a wavefront (row of NK <= 4096 bf16 / 2048 fp32 scores):
//   1. the row is loaded into registers with 16-byte loads, all in flight at once (lane l holds chunks
//      l, l+64, ...), and turned into order codes (packed 16-bit ops for bf16);
//   2. each lane's maximum code; the knn-th largest of the 64 lane maxima, code0, is reached by at least knn
//      elements (the top knn lanes each hold one), found by a bitwise search over ballot() counts;
//   3. the 16-byte chunks holding an element >= code0 are staged in LDS, and their elements >= code0 (typically a
//      few dozen) are compacted into the candidate list via a lane prefix sum;
//   4. up to 64 candidates (the usual case: one per lane) are sorted by a register bitonic network and the first
//      knn lanes are the answer; more candidates take the same bitwise search for the exact knn-th largest key t1,
//      with the knn keys >= t1 compacted and put in descending order by counting ranks.
// Rows outside the register shapes, or with more than kCap elements at or above code0 (adversarial ties),
// take the streaming path, which searches the row in global memory directly.
#include "pkm_bag_dev.h"
#include "pkm_common.h"

namespace smlm {
namespace {

constexpr int kCap = 1024;       // LDS candidates per half
constexpr int kRegCand = 4;      // candidates per lane held in registers for the exact search (C <= 256)
constexpr int kMaxKnn = 64;      // power-of-two knn up to this: the constant pair table, one result per lane
constexpr int kMaxKnnGen = 128;  // any other knn up to this: pairs built at run time, two results per lane
constexpr int kGenPairSlots = 11;  // pairs of knn = 128: sum_{i=1}^{128} floor(128 / i) = 645 <= 11 * 64

// Bits of a sub-key index below NK (any NK >= 1) and of a table index below NK^2: the bits of a key's index field
// above these are set in every key (the field holds 2^B - 1 - index).
__device__ __host__ __forceinline__ int index_bits(int NK) { return NK <= 1 ? 0 : 32 - __builtin_clz((uint32_t)NK - 1); }
__device__ __host__ __forceinline__ int pair_bits(int NK) {
  return NK <= 1 ? 0 : 64 - __builtin_clzll((uint64_t)NK * (uint64_t)NK - 1);
}

// ---- the Cartesian pair list, built at compile time: for knn = 2^lg, pairs [off[lg], off[lg+1]) ------------
// Pair p of knn = 2^lg is ij[off[lg] + p] = i | j << 8; entries past the list read as kNoPair.
constexpr uint32_t kNoPair = 0xFFFFu;
constexpr int kMaxPairSlots = 5;  // ceil(280 / 64)
struct PairTable {
  uint32_t off[8];
  uint16_t ij[481 + kMaxPairSlots * 64];
};
constexpr PairTable make_pairs() {
  PairTable t{};
  int n = 0;
  for (int lg = 0; lg <= 6; ++lg) {
    const int knn = 1 << lg;
    t.off[lg] = (uint32_t)n;
    for (int i = 0; i < knn; ++i)
      for (int j = 0; (i + 1) * (j + 1) <= knn; ++j) t.ij[n++] = (uint16_t)(i | (j << 8));
  }
  t.off[7] = (uint32_t)n;  // 1 + 3 + 8 + 20 + 50 + 119 + 280 = 481
  for (int p = n; p < 481 + kMaxPairSlots * 64; ++p) t.ij[p] = (uint16_t)kNoPair;
  return t;
}
__constant__ PairTable kPairs = make_pairs();

// This lane's Cartesian pairs for knn (slot s: pair s * 64 + lane, or kNoPair past the list), loaded at kernel
// start so that the Cartesian step, after the half selections, does not wait on memory.
__device__ __forceinline__ void load_pairs(int knn, uint32_t (&pc)[kMaxPairSlots]) {
  const int lg = 31 - __builtin_clz(knn);
  const int base = (int)kPairs.off[lg], P = (int)kPairs.off[lg + 1] - base;
  const int lane = lane_id();
#pragma unroll
  for (int s = 0; s < kMaxPairSlots; ++s) {
    const int p = s * kWave + lane;
    pc[s] = p < P ? kPairs.ij[base + p] : kNoPair;
  }
}

template <bool F32> struct SelKey;
template <> struct SelKey<false> { using T = uint32_t; };
template <> struct SelKey<true> { using T = uint64_t; };

template <bool F32>
__device__ __forceinline__ typename SelKey<F32>::T make_key(uint32_t code, uint32_t k) {
  if constexpr (F32) return ((uint64_t)code << 32) | (uint64_t)(0xFFFFFFFFu - k);
  else return (code << 16) | (0xFFFFu - k);
}
template <bool F32>
__device__ __forceinline__ typename SelKey<F32>::T half_key(const void *row, int k) {
  if constexpr (F32) return make_key<true>(order32(((const uint32_t *)row)[k]), (uint32_t)k);
  else return make_key<false>(order16(((const uint16_t *)row)[k]), (uint32_t)k);
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

// Largest t with count_ge(t) >= need, searching bits [0, bits) (count_ge is wave-uniform, non-increasing in t,
// count_ge(0) >= need, and no key has bits at or above `bits`).
template <typename Key, typename CountGE>
__device__ __forceinline__ Key threshold_search(int need, int bits, CountGE count_ge) {
  Key t = 0;
  for (int b = bits - 1; b >= 0; --b) {
    const Key c = t | ((Key)1 << b);
    if (count_ge(c) >= need) t = c;
  }
  return t;
}

// The same search over keys (code << S) | ((2^S - 1) - index) with index < 2^IB and codes in bits [S, top): bits
// [IB, S) are set in every key, so the knn-th largest key has them too and they are set without a test; only the
// code bits and the IB index bits are searched.
template <typename Key, typename CountGE>
__device__ __forceinline__ Key key_search(int need, int top, int S, int IB, CountGE count_ge) {
  Key t = 0;
  for (int b = top - 1; b >= S; --b) {
    const Key c = t | ((Key)1 << b);
    if (count_ge(c) >= need) t = c;
  }
  t |= (((Key)1 << S) - 1) & ~(((Key)1 << IB) - 1);
  for (int b = IB - 1; b >= 0; --b) {
    const Key c = t | ((Key)1 << b);
    if (count_ge(c) >= need) t = c;
  }
  return t;
}

// Number of this wavefront's lanes whose key is >= c (c >= 1: lanes holding key 0 never count).
template <typename Key>
__device__ __forceinline__ int count_ge_lanes(Key v, Key c) {
  return (int)__popcll(__builtin_amdgcn_ballot_w64(v >= c));
}

// rank of u among the n keys of sel[] (n a multiple of 4, zero keys past the real ones): how many are larger;
// 16-byte reads
template <typename Key>
__device__ __forceinline__ int rank_in(const Key *sel, int n, Key u) {
  constexpr int PER = 16 / (int)sizeof(Key);
  int rank = 0;
  for (int j0 = 0; j0 < n; j0 += 2 * PER) {
    const uint4 a = *(const uint4 *)(sel + j0), b = *(const uint4 *)(sel + j0 + PER);
    const Key *ka = (const Key *)&a, *kb = (const Key *)&b;
#pragma unroll
    for (int e = 0; e < PER; ++e) rank += (ka[e] > u) + (j0 + PER + e < n && kb[e] > u);
  }
  return rank;
}

// Exclusive prefix sum over the wavefront with DPP (shifts within 16-lane rows, then row broadcasts of lanes 15 and
// 31), no LDS round trips; *total = the sum over all lanes.  All 64 lanes must be active.
__device__ __forceinline__ int wave_exclusive_sum(int v, int *total) {
  int incl = v;
  incl += __builtin_amdgcn_update_dpp(0, incl, 0x111, 0xF, 0xF, true);   // row_shr:1
  incl += __builtin_amdgcn_update_dpp(0, incl, 0x112, 0xF, 0xF, true);   // row_shr:2
  incl += __builtin_amdgcn_update_dpp(0, incl, 0x114, 0xF, 0xF, true);   // row_shr:4
  incl += __builtin_amdgcn_update_dpp(0, incl, 0x118, 0xF, 0xF, true);   // row_shr:8
  incl += __builtin_amdgcn_update_dpp(0, incl, 0x142, 0xA, 0xF, false);  // row_bcast:15 into rows 1, 3
  incl += __builtin_amdgcn_update_dpp(0, incl, 0x143, 0xC, 0xF, false);  // row_bcast:31 into rows 2, 3
  *total = __builtin_amdgcn_readlane(incl, kWave - 1);
  return incl - v;
}

// v of lane ^ J for a 32- or 64-bit key
template <int J, typename Key>
__device__ __forceinline__ Key xor_lane_key(Key v) {
  if constexpr (sizeof(Key) == 8) return xor_lane64<J>(v);
  else return xor_lane<J>(v);
}

// (v[lane & ~J], v[lane | J]) on every lane for J = 16, 32: the gfx950 permlane swaps of a register with itself
// return the lower lane's value in their first result and the upper lane's in their second
template <int J>
__device__ __forceinline__ void lane_pair(uint32_t v, uint32_t &lo, uint32_t &hi) {
  const auto p = J == 16 ? __builtin_amdgcn_permlane16_swap(v, v, false, false)
                         : __builtin_amdgcn_permlane32_swap(v, v, false, false);
  lo = (uint32_t)p[0];
  hi = (uint32_t)p[1];
}
template <int J>
__device__ __forceinline__ void lane_pair(uint64_t v, uint64_t &lo, uint64_t &hi) {
  uint32_t l0, h0, l1, h1;
  lane_pair<J>((uint32_t)v, l0, h0);
  lane_pair<J>((uint32_t)(v >> 32), l1, h1);
  lo = ((uint64_t)l1 << 32) | l0;
  hi = ((uint64_t)h1 << 32) | h0;
}

template <int N>
struct IntC {
  static constexpr int value = N;
};
template <int N, int I = 0, class F>
__device__ __forceinline__ void static_for(F &&f) {
  if constexpr (I < N) {
    f(IntC<I>{});
    static_for<N, I + 1>(f);
  }
}

// The lanes of slot s that keep the larger key of their pair at stage (K, J) of a descending bitonic sort: element
// e = s * 64 + lane takes the maximum when it is the lower element of a descending block or the upper element of an
// ascending one.  A constant per slot and stage.
constexpr uint64_t take_max_lanes(int K, int J, int s) {
  uint64_t m = 0;
  for (int l = 0; l < kWave; ++l) {
    const int e = s * kWave + l;
    if (((e & J) == 0) == ((e & K) == 0)) m |= (uint64_t)1 << l;
  }
  return m;
}

// One compare-exchange stage (block size K, distance J < 64) of a descending bitonic sort of the wavefront's
// SLOTS * 64 keys, element e = s * 64 + lane.  Each lane holds a pair (a, b) of its key and its partner's and keeps
// a where (a > b) equals its take-max bit: the compare writes a lane mask, one scalar xnor with the stage's constant
// mask turns it into the select's, so a stage costs the lane exchange, one compare and one select per 32-bit word
// (the lane-dependent direction computed per lane cost three more vector instructions per stage: the config-2
// selection measured 146 -> 129 us with this form, the selection being bound by vector-instruction issue).  J = 16,
// 32: the pair comes from the permlane swap as (lower lane's key, upper lane's key), which needs no select to recover
// the partner.
template <typename Key, int SLOTS, int K, int J>
__device__ __forceinline__ void bitonic_stage(Key (&x)[SLOTS]) {
  static_for<SLOTS>([&](auto sc) {
    constexpr int s = decltype(sc)::value;
    constexpr uint64_t tm = take_max_lanes(K, J, s);
    Key a, b;
    if constexpr (J == 16 || J == 32) {
      lane_pair<J>(x[s], a, b);
    } else {
      a = x[s];
      b = xor_lane_key<J>(x[s]);
    }
    const uint64_t keep = ~(__builtin_amdgcn_ballot_w64(a > b) ^ tm);
    x[s] = __builtin_amdgcn_inverse_ballot_w64(keep) ? a : b;
  });
}

template <typename Key, int SLOTS, int K, int J>
__device__ __forceinline__ void bitonic_merge(Key (&x)[SLOTS]) {
  if constexpr (J >= kWave) {  // partner in the same lane: slots s and s ^ (J / 64)
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) {
      const int s2 = s ^ (J / kWave);
      if (s2 > s) {
        const bool desc = ((s * kWave) & K) == 0;
        const Key a = x[s], b = x[s2];
        const Key mx = a > b ? a : b, mn = a > b ? b : a;
        x[s] = desc ? mx : mn;
        x[s2] = desc ? mn : mx;
      }
    }
  } else {
    bitonic_stage<Key, SLOTS, K, J>(x);
  }
  if constexpr (J > 1) bitonic_merge<Key, SLOTS, K, J / 2>(x);
}

// Descending bitonic sort of SLOTS * 64 unique keys held one per lane per slot; afterwards lane j of slot 0 holds
// the j-th largest.
template <typename Key, int SLOTS, int K = 2>
__device__ __forceinline__ void bitonic_sort_desc(Key (&x)[SLOTS]) {
  bitonic_merge<Key, SLOTS, K, K / 2>(x);
  if constexpr (K < SLOTS * kWave) bitonic_sort_desc<Key, SLOTS, K * 2>(x);
}

// The knn keys >= t (exactly knn exist) from `src` (n entries, LDS) into out[] in descending order; sel[] and out[]
// hold MAXK keys.
template <typename Key, int MAXK, typename Fetch>
__device__ __forceinline__ void collect_sorted(int n, int knn, Key t, Fetch fetch, Key *sel, Key *out) {
  const int lane = lane_id();
  int S = 0;
  for (int p0 = 0; p0 < n; p0 += kWave) {
    const int p = p0 + lane;
    const Key u = p < n ? fetch(p) : (Key)0;
    const bool ge = p < n && u >= t;
    const uint64_t m = ballot(ge);
    const int pos = S + lanes_below(m);
    if (ge && pos < MAXK) sel[pos] = u;
    S += (int)__popcll(m);
  }
  if constexpr (MAXK <= kWave) {
    if (lane >= knn && lane < 4) sel[lane] = 0;     // pad knn < 4 to whole 16-byte reads
    wave_lds_sync();
    if (lane < knn) {
      const Key u = sel[lane];
      out[rank_in(sel, knn < 4 ? 4 : knn, u)] = u;
    }
  } else {
    const int padded = (knn + 7) & ~7;              // zero keys up to whole pairs of 16-byte reads
    for (int q = knn + lane; q < padded; q += kWave) sel[q] = 0;
    wave_lds_sync();
    for (int q = lane; q < knn; q += kWave) {
      const Key u = sel[q];
      out[rank_in(sel, padded, u)] = u;
    }
  }
  wave_lds_sync();
}

// Exact top-knn among C candidate keys in LDS (keys of sub-key indices < 2^IB), into out[] descending.
template <bool F32, int MAXK>
__device__ __forceinline__ void topk_of_candidates(int C, int knn, int IB, typename SelKey<F32>::T *cand,
                                                   typename SelKey<F32>::T *sel, typename SelKey<F32>::T *out) {
  using Key = typename SelKey<F32>::T;
  constexpr int kTop = F32 ? 64 : 32, kS = F32 ? 32 : 16;
  const int lane = lane_id();
  Key t;
  if (C <= kWave) {  // one key per lane (the common case): sort them, the first knn lanes are the answer
    Key x[1] = {lane < C ? cand[lane] : (Key)0};
    bitonic_sort_desc<Key, 1>(x);
    if (lane < knn) out[lane] = x[0];
    wave_lds_sync();
    return;
  } else if (C <= kRegCand * kWave) {
    Key reg[kRegCand];
#pragma unroll
    for (int s = 0; s < kRegCand; ++s) {
      const int p = s * kWave + lane;
      reg[s] = p < C ? cand[p] : (Key)0;
    }
    t = key_search<Key>(knn, kTop, kS, IB, [&](Key c) {
      int n = 0;
#pragma unroll
      for (int s = 0; s < kRegCand; ++s) n += count_ge_lanes(reg[s], c);
      return n;
    });
  } else {
    t = key_search<Key>(knn, kTop, kS, IB, [&](Key c) {
      int n = 0;
      for (int p0 = 0; p0 < C; p0 += kWave) {
        const int p = p0 + lane;
        n += count_ge_lanes(p < C ? cand[p] : (Key)0, c);
      }
      return n;
    });
  }
  collect_sorted<Key, MAXK>(C, knn, t, [&](int p) { return cand[p]; }, sel, out);
}

// Streaming half top-k: any NK, searching the row in global memory.  Up to 64 lanes, the knn-th largest lane maximum
// bounds the answer from below; a larger knn takes every element as a candidate (or, past the LDS, the exact search
// over the row).
template <bool F32, int CAP, int MAXK>
__device__ void half_topk_stream(const void *row, int NK, int knn, typename SelKey<F32>::T *cand,
                                 typename SelKey<F32>::T *sel, typename SelKey<F32>::T *out) {
  using Key = typename SelKey<F32>::T;
  constexpr int kBits = F32 ? 64 : 32;
  const int lane = lane_id();
  Key t0 = 0;
  if (knn <= kWave) {
    Key mx = 0;
    for (int k = lane; k < NK; k += kWave) {
      const Key u = half_key<F32>(row, k);
      mx = u > mx ? u : mx;
    }
    t0 = threshold_search<Key>(knn, kBits, [&](Key t) { return count_ge_lanes(mx, t); });
  }
  int C = 0;
  for (int k0 = 0; k0 < NK; k0 += kWave) {
    const int k = k0 + lane;
    const Key u = k < NK ? half_key<F32>(row, k) : (Key)0;
    const bool take = k < NK && u >= t0;
    const uint64_t m = ballot(take);
    const int pos = C + lanes_below(m);
    if (take && pos < CAP) cand[pos] = u;
    C += (int)__popcll(m);
  }
  wave_lds_sync();
  if (C <= CAP) {
    topk_of_candidates<F32, MAXK>(C, knn, index_bits(NK), cand, sel, out);
    return;
  }
  const Key t1 = threshold_search<Key>(knn, kBits, [&](Key t) {
    int cnt = 0;
    for (int k0 = 0; k0 < NK; k0 += kWave) {
      const int k = k0 + lane;
      cnt += count_ge_lanes(k < NK ? half_key<F32>(row, k) : (Key)0, t);
    }
    return cnt;
  });
  collect_sorted<Key, MAXK>(NK, knn, t1, [&](int k) { return half_key<F32>(row, k); }, sel, out);
}

typedef short s16x2 __attribute__((ext_vector_type(2)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

// order codes of one 16-byte chunk, in place: bf16 -> two 16-bit codes per dword; fp32 -> one code per dword
template <bool F32>
__device__ __forceinline__ uint4 chunk_codes(uint4 v) {
  uint32_t d[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    if constexpr (F32) {
      d[e] ^= (uint32_t)((int32_t)d[e] >> 31) | 0x80000000u;
    } else {
      const s16x2 sgn = __builtin_bit_cast(s16x2, d[e]) >> (short)15;  // 0xFFFF where negative
      d[e] ^= __builtin_bit_cast(uint32_t, sgn) | 0x80008000u;
    }
  }
  return uint4{d[0], d[1], d[2], d[3]};
}

// Register half top-k for NK = CPL * 64 chunks of 16 bytes (or fewer chunks, down to one):
//   1. the row into registers as order codes (lane l holds chunks l, l + 64, ...), with each chunk's largest code;
//   2. code0 = the knn-th largest lane maximum: at least knn elements reach it (the top knn lanes hold one each);
//   3. the chunks whose maximum reaches code0 (a few dozen) are staged in LDS, one per lane per round, so that
//   4. each lane appends only its staged chunk's elements >= code0 to the candidate list (DPP prefix sum);
//   5. the exact top knn of the candidates, in descending order.
// The wavefront's CAP keys of LDS hold the candidates at the front and the staging area (16 bytes + chunk index
// per lane) at the back; a row with more candidates than fit takes the streaming path.
template <bool F32, int CPL, int CAP, int MAXK>
__device__ __forceinline__ void half_topk_reg(const void *row, int NK, int knn, typename SelKey<F32>::T *cand,
                                              typename SelKey<F32>::T *sel, typename SelKey<F32>::T *out) {
  using Key = typename SelKey<F32>::T;
  constexpr int EPC = F32 ? 4 : 8;  // elements per chunk
  constexpr int kStageBytes = kWave * (16 + 4);
  constexpr int kCandMax = (CAP * (int)sizeof(Key) - kStageBytes) / (int)sizeof(Key);
  static_assert(kCandMax >= MAXK, "candidate area too small");
  uint4 *stage = (uint4 *)((char *)cand + CAP * sizeof(Key) - kStageBytes);
  uint32_t *stage_id = (uint32_t *)(stage + kWave);
  const int lane = lane_id();
  const int nchunks = NK / EPC;

  uint4 code[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int c = lane + j * kWave;
    code[j] = c < nchunks ? ((const uint4 *)row)[c] : uint4{0u, 0u, 0u, 0u};
  }
  uint32_t cmax[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int c = lane + j * kWave;
    code[j] = c < nchunks ? chunk_codes<F32>(code[j]) : uint4{0u, 0u, 0u, 0u};  // invalid -> code 0 (minimum)
    if constexpr (F32) {
      cmax[j] = max(max(code[j].x, code[j].y), max(code[j].z, code[j].w));
    } else {
      u16x2 pm = __builtin_elementwise_max(__builtin_bit_cast(u16x2, code[j].x), __builtin_bit_cast(u16x2, code[j].y));
      pm = __builtin_elementwise_max(pm, __builtin_bit_cast(u16x2, code[j].z));
      pm = __builtin_elementwise_max(pm, __builtin_bit_cast(u16x2, code[j].w));
      cmax[j] = max((uint32_t)pm.x, (uint32_t)pm.y);
    }
  }
  uint32_t mx = 0;
#pragma unroll
  for (int j = 0; j < CPL; ++j) mx = max(mx, cmax[j]);
  const uint32_t code0 = threshold_search<uint32_t>(knn, F32 ? 32 : 16,
                                                    [&](uint32_t t) { return count_ge_lanes(mx, t); });

  // candidate chunks: per slot j a ballot, numbered slot by slot in lane order
  uint64_t bm[CPL];
  int base[CPL];
  int Cc = 0;
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    bm[j] = ballot(lane + j * kWave < nchunks && cmax[j] >= code0);
    base[j] = Cc;
    Cc += (int)__popcll(bm[j]);
  }
  int C = 0;
  for (int r0 = 0; r0 < Cc; r0 += kWave) {  // one round unless more than 64 chunks reach code0
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const int p = base[j] + lanes_below(bm[j]) - r0;
      if (((bm[j] >> lane) & 1) && p >= 0 && p < kWave) {
        stage[p] = code[j];
        stage_id[p] = (uint32_t)(lane + j * kWave);
      }
    }
    wave_lds_sync();
    const bool have = r0 + lane < Cc;
    const uint4 v = have ? stage[lane] : uint4{0u, 0u, 0u, 0u};
    const uint32_t cid = have ? stage_id[lane] : 0u;
    const uint32_t d[4] = {v.x, v.y, v.z, v.w};
    uint32_t ec[EPC];
    int n = 0;
#pragma unroll
    for (int e = 0; e < EPC; ++e) {
      if constexpr (F32) ec[e] = d[e];
      else ec[e] = (d[e >> 1] >> (16 * (e & 1))) & 0xFFFFu;
      n += (have && ec[e] >= code0) ? 1 : 0;
    }
    int total;
    int pos = C + wave_exclusive_sum(n, &total);
    if (C + total <= kCandMax) {
#pragma unroll
      for (int e = 0; e < EPC; ++e)
        if (have && ec[e] >= code0) cand[pos++] = make_key<F32>(ec[e], cid * EPC + (uint32_t)e);
    }
    C += total;
    wave_lds_sync();  // the staging area is rewritten by the next round
  }
  if (C <= kCandMax) {
    topk_of_candidates<F32, MAXK>(C, knn, index_bits(NK), cand, sel, out);
  } else {
    half_topk_stream<F32, CAP, MAXK>(row, NK, knn, cand, sel, out);
  }
}

// Sum over the wavefront: DPP sums within each 16-lane row, then the four row totals.  All lanes active.
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false));
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
  return (r0 + r1) + (r2 + r3);
}

// The Cartesian pairs' keys (code << 32 | ~full index; 0 for a slot without a pair)
template <bool F32, int SLOTS>
__device__ __forceinline__ void cartesian_keys(const typename SelKey<F32>::T *top1, const typename SelKey<F32>::T *top2,
                                               int NK, const uint32_t (&pc)[kMaxPairSlots], uint64_t (&ck)[SLOTS]) {
  using Key = typename SelKey<F32>::T;
#pragma unroll
  for (int s = 0; s < SLOTS; ++s) {
    ck[s] = 0;
    if (pc[s] != kNoPair) {
      const Key k1 = top1[pc[s] & 0xFFu];
      const Key k2 = top2[pc[s] >> 8];
      const float sum = key_value<F32>(k1) + key_value<F32>(k2);
      const uint32_t code = F32 ? order32(__float_as_uint(sum)) : order16(bf16_bits_rtne(sum));
      const uint32_t full = key_index<F32>(k1) * (uint32_t)NK + key_index<F32>(k2);
      ck[s] = ((uint64_t)code << 32) | (uint64_t)(0xFFFFFFFFu - full);
    }
  }
}

template <bool F32, int SLOTS>
__device__ __forceinline__ uint64_t cartesian_threshold(const typename SelKey<F32>::T *top1,
                                                        const typename SelKey<F32>::T *top2, int NK, int knn,
                                                        const uint32_t (&pc)[kMaxPairSlots], uint64_t *s_fsel) {
  using Key = typename SelKey<F32>::T;
  uint64_t ck[SLOTS];
#pragma unroll
  for (int s = 0; s < SLOTS; ++s) {
    ck[s] = 0;  // no pair: key 0, never counted (every tested threshold is >= 1)
    if (pc[s] != kNoPair) {
      const Key k1 = top1[pc[s] & 0xFFu];
      const Key k2 = top2[pc[s] >> 8];
      const float sum = key_value<F32>(k1) + key_value<F32>(k2);
      const uint32_t code = F32 ? order32(__float_as_uint(sum)) : order16(bf16_bits_rtne(sum));
      const uint32_t full = key_index<F32>(k1) * (uint32_t)NK + key_index<F32>(k2);
      ck[s] = ((uint64_t)code << 32) | (uint64_t)(0xFFFFFFFFu - full);
    }
  }
  // table indices are below NK^2 <= 2^IB: the bits above them in the low word are set in every key
  const int IB = pair_bits(NK);
  const uint64_t t = key_search<uint64_t>(knn, F32 ? 64 : 48, 32, IB, [&](uint64_t c) {
    int n = 0;
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) n += count_ge_lanes(ck[s], c);
    return n;
  });
  int S = 0;
#pragma unroll
  for (int s = 0; s < SLOTS; ++s) {
    const bool ge = ck[s] >= t;  // t >= 1: pair-less slots never qualify
    const uint64_t m = __builtin_amdgcn_ballot_w64(ge);
    const int pos = S + lanes_below(m);
    if (ge && pos < kMaxKnn) s_fsel[pos] = ck[s];
    S += (int)__popcll(m);
  }
  return t;
}

// Cartesian step of one head: candidates (i, j) with (i+1)(j+1) <= knn of the two halves' descending top lists,
// scored dtype(v1[i] + v2[j]), top-knn by (score, lowest table index), softmax in fp32.  Called by both wavefronts
// of the head, p = 0 and p = 1 (and by every wavefront of the workgroup, since knn = 32 has a workgroup barrier);
// returns true on wavefront 0, whose lane j < knn then holds the j-th best pair: its score `sc` (code = order code of
// its bits), table index `full` and weight `wt`.  pc: the lane's pairs from load_pairs; s_x, s_fsel, s_fin: kMaxKnn
// entries of LDS scratch each (s_x may be s_fin).
// Pairs per knn: <= 50 (one slot of 64 lanes), 119 (two), 280 (five).  One slot: a bitonic sort in registers (keys
// are unique: distinct pairs have distinct table indices; pair-less slots sort last).  Two slots: each wavefront
// sorts one, wavefront 1 leaves its sorted keys in s_x, and wavefront 0 takes, lane by lane, the larger of its j-th
// and the other's (63 - j)-th key: the 64 largest of both, a bitonic sequence, which one merge puts in order.
// Five: the threshold search, compaction and rank through LDS.
template <bool F32>
__device__ __forceinline__ bool cartesian_topk(const typename SelKey<F32>::T *top1,
                                               const typename SelKey<F32>::T *top2, int NK, int knn,
                                               const uint32_t (&pc)[kMaxPairSlots], int p, uint64_t *s_x,
                                               uint64_t *s_fsel, uint64_t *s_fin, float &sc, uint32_t &full,
                                               uint32_t &code, float &wt) {
  const int lane = lane_id();
  uint64_t u = 0;
  if (knn == 32) {
    const uint32_t mine[kMaxPairSlots] = {pc[p], kNoPair, kNoPair, kNoPair, kNoPair};
    uint64_t x[1];
    cartesian_keys<F32, 1>(top1, top2, NK, mine, x);
    bitonic_sort_desc<uint64_t, 1>(x);
    if (p == 1) s_x[lane] = x[0];
    __syncthreads();
    if (p != 0) return false;
    const uint64_t y = s_x[kWave - 1 - lane];
    uint64_t m[1] = {x[0] > y ? x[0] : y};
    bitonic_merge<uint64_t, 1, kWave, kWave / 2>(m);
    u = m[0];
  } else {
    if (p != 0) return false;
    if (knn >= 64) {
      cartesian_threshold<F32, 5>(top1, top2, NK, knn, pc, s_fsel);
      wave_lds_sync();
      if (lane < knn) {
        const uint64_t mine = s_fsel[lane];
        s_fin[rank_in(s_fsel, knn, mine)] = mine;
      }
      wave_lds_sync();
      if (lane < knn) u = s_fin[lane];
    } else {
      uint64_t ck[1];
      cartesian_keys<F32, 1>(top1, top2, NK, pc, ck);
      bitonic_sort_desc<uint64_t, 1>(ck);
      u = ck[0];
    }
  }

  sc = 0.f;
  full = 0;
  code = 0;
  if (lane < knn) {
    code = (uint32_t)(u >> 32);
    full = 0xFFFFFFFFu - (uint32_t)u;
    sc = F32 ? __uint_as_float(unorder32(code)) : bf16_bits_to_f32(unorder16(code));
  }
  // descending: lane 0 holds the largest score
  const float mxs = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sc), 0));
  const float e = lane < knn ? expf(sc - mxs) : 0.f;
  wt = e / wave_sum_dpp(e);
  return true;
}


// ---- any knn up to kMaxKnnGen: the pair list built at run time, two results per lane ----------------------------
// Pairs (i, j) with (i + 1)(j + 1) <= knn in row order: pair p is (i, p - pre[i]) for the row i with
// pre[i] <= p < pre[i + 1], pre[i] = sum_{r < i} floor(knn / (r + 1)) (the same list, in the same order, as the
// constant table's).  pre: the wavefront's LDS scratch of at least kMaxKnnGen + 1 ints.  Slots past the list hold
// kNoPair; returns the pair count.
__device__ __forceinline__ int gen_pairs(int knn, int *pre, uint32_t (&pc)[kGenPairSlots]) {
  const int lane = lane_id();
  int carry = 0;
  for (int r0 = 0; r0 < knn; r0 += kWave) {  // at most two rounds
    const int i = r0 + lane;
    const int c = i < knn ? knn / (i + 1) : 0;
    int total;
    const int ex = wave_exclusive_sum(c, &total);
    if (i < knn) pre[i] = carry + ex;
    carry += total;
  }
  wave_lds_sync();
  const int P = carry;
  int cur[kGenPairSlots];
#pragma unroll
  for (int s = 0; s < kGenPairSlots; ++s) cur[s] = 0;
  // the last row whose start is <= p, seven bisection steps (knn <= 128) over all slots at once
#pragma unroll
  for (int b = 6; b >= 0; --b) {
#pragma unroll
    for (int s = 0; s < kGenPairSlots; ++s) {
      const int probe = cur[s] | (1 << b);
      const int p = s * kWave + lane;
      if (probe < knn && pre[probe] <= p) cur[s] = probe;
    }
  }
#pragma unroll
  for (int s = 0; s < kGenPairSlots; ++s) {
    const int p = s * kWave + lane;
    pc[s] = p < P ? (uint32_t)cur[s] | ((uint32_t)(p - pre[cur[s]]) << 8) : kNoPair;
  }
  wave_lds_sync();
  return P;
}

// Cartesian step of one head for any knn <= kMaxKnnGen (wavefront 0 of the head only): the pairs' keys, the exact
// knn-th largest by the threshold search, the keys at or above it compacted and ranked through LDS (s_fsel, s_fin:
// kMaxKnnGen entries each), then the fp32 softmax.  Lane l holds results j = l (r = 0) and j = l + 64 (r = 1) for
// j < knn: score sc[r] (code[r] = its order code), table index full[r], weight wt[r].
template <bool F32>
__device__ __forceinline__ void cartesian_general(const typename SelKey<F32>::T *top1,
                                                  const typename SelKey<F32>::T *top2, int NK, int knn,
                                                  const uint32_t (&pc)[kGenPairSlots], uint64_t *s_fsel,
                                                  uint64_t *s_fin, float (&sc)[2], uint32_t (&full)[2],
                                                  uint32_t (&code)[2], float (&wt)[2]) {
  using Key = typename SelKey<F32>::T;
  const int lane = lane_id();
  uint64_t ck[kGenPairSlots];
#pragma unroll
  for (int s = 0; s < kGenPairSlots; ++s) {
    ck[s] = 0;  // no pair: key 0, never counted (every tested threshold is >= 1)
    if (pc[s] != kNoPair) {
      const Key k1 = top1[pc[s] & 0xFFu];
      const Key k2 = top2[pc[s] >> 8];
      const float sum = key_value<F32>(k1) + key_value<F32>(k2);
      const uint32_t cd = F32 ? order32(__float_as_uint(sum)) : order16(bf16_bits_rtne(sum));
      const uint32_t f = key_index<F32>(k1) * (uint32_t)NK + key_index<F32>(k2);
      ck[s] = ((uint64_t)cd << 32) | (uint64_t)(0xFFFFFFFFu - f);
    }
  }
  const uint64_t t = key_search<uint64_t>(knn, F32 ? 64 : 48, 32, pair_bits(NK), [&](uint64_t c) {
    int n = 0;
#pragma unroll
    for (int s = 0; s < kGenPairSlots; ++s) n += count_ge_lanes(ck[s], c);
    return n;
  });
  int S = 0;
#pragma unroll
  for (int s = 0; s < kGenPairSlots; ++s) {
    const bool ge = ck[s] >= t;
    const uint64_t m = __builtin_amdgcn_ballot_w64(ge);
    const int pos = S + lanes_below(m);
    if (ge && pos < kMaxKnnGen) s_fsel[pos] = ck[s];
    S += (int)__popcll(m);
  }
  const int padded = (knn + 3) & ~3;
  for (int q = knn + lane; q < padded; q += kWave) s_fsel[q] = 0;
  wave_lds_sync();
  for (int q = lane; q < knn; q += kWave) {
    const uint64_t mine = s_fsel[q];
    s_fin[rank_in(s_fsel, padded, mine)] = mine;
  }
  wave_lds_sync();
  float e[2];
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int j = lane + r * kWave;
    const uint64_t u = j < knn ? s_fin[j] : 0;
    code[r] = (uint32_t)(u >> 32);
    full[r] = 0xFFFFFFFFu - (uint32_t)u;
    sc[r] = j < knn ? (F32 ? __uint_as_float(unorder32(code[r])) : bf16_bits_to_f32(unorder16(code[r]))) : 0.f;
  }
  // descending: lane 0's first result is the largest score
  const float mxs = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sc[0]), 0));
#pragma unroll
  for (int r = 0; r < 2; ++r) e[r] = lane + r * kWave < knn ? expf(sc[r] - mxs) : 0.f;
  const float sum = wave_sum_dpp(e[0] + e[1]);
#pragma unroll
  for (int r = 0; r < 2; ++r) wt[r] = e[r] / sum;
}

// One workgroup (two wavefronts) per (token, head).  GEN: any knn <= kMaxKnnGen (pairs built at run time, two
// results per lane, the half top-k from the row in memory when knn > 64); otherwise a power-of-two knn <= kMaxKnn.
template <bool F32, int CPL, bool GEN>
__global__ void __launch_bounds__(128) select_kernel(const void *__restrict__ s1, const void *__restrict__ s2,
                                                     int NK, int knn, void *__restrict__ scores,
                                                     int64_t *__restrict__ idx, float *__restrict__ w) {
  using Key = typename SelKey<F32>::T;
  constexpr int MAXK = GEN ? kMaxKnnGen : kMaxKnn;
  __shared__ __align__(16) Key s_cand[2][kCap];
  __shared__ __align__(16) Key s_sel[2][MAXK];
  __shared__ __align__(16) Key s_top[2][MAXK];
  __shared__ __align__(16) uint64_t s_fsel[MAXK];
  __shared__ __align__(16) uint64_t s_fin[MAXK];

  const int wave = threadIdx.x / kWave;
  const int lane = lane_id();
  const int64_t row = blockIdx.x;  // n * H + h
  const size_t esz = F32 ? 4 : 2;
  const void *src = (const char *)(wave == 0 ? s1 : s2) + row * (int64_t)NK * esz;
  if constexpr (!GEN) {
    uint32_t pc[kMaxPairSlots];
    load_pairs(knn, pc);
    if constexpr (CPL > 0) half_topk_reg<F32, CPL, kCap, MAXK>(src, NK, knn, s_cand[wave], s_sel[wave], s_top[wave]);
    else half_topk_stream<F32, kCap, MAXK>(src, NK, knn, s_cand[wave], s_sel[wave], s_top[wave]);
    __syncthreads();

    float sc, wt;
    uint32_t full, code;
    if (!cartesian_topk<F32>(s_top[0], s_top[1], NK, knn, pc, wave, s_fin, s_fsel, s_fin, sc, full, code, wt))
      return;
    if (lane < knn) {
      const int64_t o = row * knn + lane;
      if constexpr (F32) ((float *)scores)[o] = sc;
      else ((uint16_t *)scores)[o] = (uint16_t)unorder16(code);
      idx[o] = (int64_t)full;
      w[o] = wt;
    }
  } else {
    if constexpr (CPL > 0) {
      if (knn <= kWave) half_topk_reg<F32, CPL, kCap, MAXK>(src, NK, knn, s_cand[wave], s_sel[wave], s_top[wave]);
      else half_topk_stream<F32, kCap, MAXK>(src, NK, knn, s_cand[wave], s_sel[wave], s_top[wave]);
    } else {
      half_topk_stream<F32, kCap, MAXK>(src, NK, knn, s_cand[wave], s_sel[wave], s_top[wave]);
    }
    __syncthreads();
    if (wave != 0) return;
    uint32_t pc[kGenPairSlots];
    gen_pairs(knn, (int *)s_cand[0], pc);
    float sc[2], wt[2];
    uint32_t full[2], code[2];
    cartesian_general<F32>(s_top[0], s_top[1], NK, knn, pc, s_fsel, s_fin, sc, full, code, wt);
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int j = lane + r * kWave;
      if (j < knn) {
        const int64_t o = row * knn + j;
        if constexpr (F32) ((float *)scores)[o] = sc[r];
        else ((uint16_t *)scores)[o] = (uint16_t)unorder16(code[r]);
        idx[o] = (int64_t)full[r];
        w[o] = wt[r];
      }
    }
  }
}

template <bool F32>
void launch_select(const void *s1, const void *s2, int64_t rows, int NK, int knn, void *scores, int64_t *idx,
                   float *w, hipStream_t stream) {
  const int epc = F32 ? 4 : 8;
  const bool aligned = (((uintptr_t)s1 | (uintptr_t)s2) % 16) == 0 && NK % epc == 0;
  const int chunks = NK / epc;
  const dim3 grid((unsigned)rows), block(2 * kWave);
#define SMLM_SELECT(CPL, GEN) \
  hipLaunchKernelGGL((select_kernel<F32, CPL, GEN>), grid, block, 0, stream, s1, s2, NK, knn, scores, idx, w)
  if (!is_pow2(knn) || knn > kMaxKnn) {  // the general path: register rows up to 8 chunks per lane
    if (!aligned || chunks > 8 * kWave || knn > kWave) SMLM_SELECT(0, true);
    else SMLM_SELECT(8, true);
  } else if (!aligned || chunks > 8 * kWave) SMLM_SELECT(0, false);
  else if (chunks <= kWave) SMLM_SELECT(1, false);
  else if (chunks <= 2 * kWave) SMLM_SELECT(2, false);
  else if (chunks <= 4 * kWave) SMLM_SELECT(4, false);
  else SMLM_SELECT(8, false);
#undef SMLM_SELECT
}

// ---- selection fused with the value bag (decode): one workgroup per token, 2H wavefronts ----------------------
// Wavefront (h, p) selects in s_p[n, h, :]; wavefront (h, 0) then does head h's Cartesian step and softmax and
// stages its knn lookups (row offset, weight x row scale) in LDS; finally the workgroup gathers the token's H*knn
// rows in the canonical row-slot layout of bag_rows_kernel (bag::bag_slots(cpr) slots; threads past them idle, a
// thread runs several slots when the workgroup has fewer), with twice the loads in flight per thread, adds the
// slots through LDS (over the candidate buffers, no longer needed) and applies the bag epilogue.  Same selection and the same bag additions in the same order as select_kernel followed by
// bag_rows_kernel, so the results are bit-identical; it saves the launch and the round trip of the lookups.
constexpr int kFusedCapBytes = 4096;   // LDS candidate + staging bytes per half (1024 bf16 / 512 fp32 keys)

constexpr int kFusedMaxHeads = 4;       // 2H wavefronts per workgroup

template <bool F32, int CPL, int TK, bool GEN>
__global__ void __launch_bounds__(2 * kFusedMaxHeads * kWave)
    select_bag_kernel(const void *__restrict__ s1, const void *__restrict__ s2, int H, int NK, int knn,
                      const uint8_t *__restrict__ table, int64_t rows, int D, int row_bytes, int cpr,
                      const uint16_t *__restrict__ scales, const uint16_t *__restrict__ pre, void *__restrict__ out,
                      int out_bf16, size_t union_bytes, void *__restrict__ scores, int64_t *__restrict__ idx,
                      float *__restrict__ w) {
  using Key = typename SelKey<F32>::T;
  constexpr int CAP = kFusedCapBytes / (int)sizeof(Key);
  constexpr int VPC = bag::vals_per_chunk<TK>();
  constexpr int MAXK = GEN ? kMaxKnnGen : kMaxKnn;
  extern __shared__ __align__(16) unsigned char smem[];
  const int nw = 2 * H;
  Key *s_cand = (Key *)smem;                            // [nw][CAP]; then float [rpr][D] partial sums
  Key *s_sel = (Key *)(smem + union_bytes);             // [nw][MAXK]
  Key *s_top = s_sel + nw * MAXK;                       // [nw][MAXK]
  uint64_t *s_fsel = (uint64_t *)(s_top + nw * MAXK);   // [H][MAXK]
  uint64_t *s_fin = s_fsel + H * MAXK;                  // [H][MAXK]
  int64_t *s_off = (int64_t *)(s_fin + H * MAXK);       // [H * knn]
  float *s_w = (float *)(s_off + H * knn);              // [H * knn]
  __shared__ int s_bad;

  const int tid = threadIdx.x, wave = tid / kWave, lane = lane_id();
  const int h = wave >> 1, p = wave & 1;
  const int64_t n = blockIdx.x;
  const int64_t row = n * H + h;
  const size_t esz = F32 ? 4 : 2;
  if (tid == 0) s_bad = 0;
  // the swilu input of the first output column this thread stores, loaded now: read at the end it would add a
  // memory round trip after the gather
  const uint16_t pre_first = pre && tid < D ? pre[n * D + tid] : (uint16_t)0;
  const void *src = (const char *)(p ? s2 : s1) + row * (int64_t)NK * esz;
  Key *sel = s_sel + wave * MAXK, *top = s_top + wave * MAXK;

  // result j of head h (wavefront (h, 0)): outputs, and the lookup staged for the gather
  auto emit = [&](int j, float sc, uint32_t full, uint32_t code, float wt) {
    const int64_t o = row * knn + j;
    if (scores) {
      if constexpr (F32) ((float *)scores)[o] = sc;
      else ((uint16_t *)scores)[o] = (uint16_t)unorder16(code);
    }
    if (idx) idx[o] = (int64_t)full;
    if (w) w[o] = wt;
    int64_t r = full;
    float ww = wt;
    if (r >= rows) {  // a table with fewer than NK^2 rows: the token's output is NaN, as in the bag
      s_bad = 1;
      r = 0;
      ww = 0.f;
    }
    if constexpr (TK == bag::kI8 || TK == bag::kQ4) ww *= f16_bits_to_f32(scales[r]);
    s_off[h * knn + j] = r * row_bytes;
    s_w[h * knn + j] = ww;
  };

  if constexpr (!GEN) {
    uint32_t pc[kMaxPairSlots];
    load_pairs(knn, pc);
    if constexpr (CPL > 0) half_topk_reg<F32, CPL, CAP, MAXK>(src, NK, knn, s_cand + wave * CAP, sel, top);
    else half_topk_stream<F32, CAP, MAXK>(src, NK, knn, s_cand + wave * CAP, sel, top);
    __syncthreads();

    float sc, wt;
    uint32_t full, code;
    if (cartesian_topk<F32>(s_top + 2 * h * MAXK, s_top + (2 * h + 1) * MAXK, NK, knn, pc, p, s_fin + h * MAXK,
                            s_fsel + h * MAXK, s_fin + h * MAXK, sc, full, code, wt)) {
      if (lane < knn) emit(lane, sc, full, code, wt);
    }
  } else {
    if constexpr (CPL > 0) {
      if (knn <= kWave) half_topk_reg<F32, CPL, CAP, MAXK>(src, NK, knn, s_cand + wave * CAP, sel, top);
      else half_topk_stream<F32, CAP, MAXK>(src, NK, knn, s_cand + wave * CAP, sel, top);
    } else {
      half_topk_stream<F32, CAP, MAXK>(src, NK, knn, s_cand + wave * CAP, sel, top);
    }
    __syncthreads();
    if (p == 0) {
      uint32_t pc[kGenPairSlots];
      gen_pairs(knn, (int *)(s_cand + wave * CAP), pc);
      float sc[2], wt[2];
      uint32_t full[2], code[2];
      cartesian_general<F32>(s_top + 2 * h * MAXK, s_top + (2 * h + 1) * MAXK, NK, knn, pc, s_fsel + h * MAXK,
                             s_fin + h * MAXK, sc, full, code, wt);
#pragma unroll
      for (int r = 0; r < 2; ++r)
        if (lane + r * kWave < knn) emit(lane + r * kWave, sc[r], full[r], code[r], wt[r]);
    }
  }
  __syncthreads();

  // the canonical slots of the bag layout; with fewer whole slots of threads than that, a thread runs several
  const int rpr = bag::bag_slots(cpr), tslots = (int)blockDim.x / cpr, slot = tid / cpr, c = tid % cpr;
  float *s_red = (float *)smem;
  if (slot < tslots) {
    for (int cs = slot; cs < rpr; cs += tslots) {
      float acc[VPC];
#pragma unroll
      for (int e = 0; e < VPC; ++e) acc[e] = 0.f;
      bag::accumulate_rows<TK, 2 * bag::kUnroll>(table + (int64_t)c * 16, cs, rpr, H * knn, s_off, s_w, acc);
#pragma unroll
      for (int e = 0; e < VPC; ++e) s_red[cs * D + bag::chunk_col<TK>(c, e, D)] = acc[e];
    }
  }
  __syncthreads();
  const bool bad = s_bad != 0;
  for (int col = tid; col < D; col += blockDim.x) {
    float a = 0.f;
    for (int r = 0; r < rpr; ++r) a += s_red[r * D + col];
    const uint16_t pb = col == tid ? pre_first : pre ? pre[n * D + col] : (uint16_t)0;
    bag::store_out_bits(out, n * D + col, a, bad, pre != nullptr, pb, out_bf16 != 0);
  }
}

template <bool F32, int TK>
void launch_select_bag(const void *s1, const void *s2, int64_t N, int H, int NK, int knn, const void *table,
                       int64_t rows, int D, const uint16_t *scales, const uint16_t *pre, void *out, int out_bf16,
                       void *scores, int64_t *idx, float *w, hipStream_t stream) {
  using Key = typename SelKey<F32>::T;
  const bool gen = !is_pow2(knn) || knn > kMaxKnn;
  const int maxk = gen ? kMaxKnnGen : kMaxKnn;
  const int row_bytes = TK == bag::kF32 ? 4 * D : TK == bag::kBF16 ? 2 * D : TK == bag::kI8 ? D : D / 2;
  const int cpr = row_bytes / 16;
  const int nthr = 2 * H * kWave;
  const int rpr = bag::bag_slots(cpr);
  const size_t cand = (size_t)2 * H * kFusedCapBytes, red = (size_t)rpr * D * sizeof(float);
  const size_t union_bytes = (cand > red ? cand : red + 15) / 16 * 16;
  const size_t shmem = union_bytes + (size_t)2 * 2 * H * maxk * sizeof(Key) + (size_t)2 * H * maxk * 8 +
                       (size_t)H * knn * (8 + 4);
  const int epc = F32 ? 4 : 8;
  const bool aligned = (((uintptr_t)s1 | (uintptr_t)s2) % 16) == 0 && NK % epc == 0;
  const int chunks = NK / epc;
  const dim3 grid((unsigned)N), block(nthr);
#define SMLM_SELECT_BAG(CPL, GEN)                                                                                \
  hipLaunchKernelGGL((select_bag_kernel<F32, CPL, TK, GEN>), grid, block, shmem, stream, s1, s2, H, NK, knn,     \
                     (const uint8_t *)table, rows, D, row_bytes, cpr, scales, pre, out, out_bf16, union_bytes, \
                     scores, idx, w)
  if (gen) {
    if (!aligned || chunks > 8 * kWave || knn > kWave) SMLM_SELECT_BAG(0, true);
    else SMLM_SELECT_BAG(8, true);
  } else if (!aligned || chunks > 8 * kWave) SMLM_SELECT_BAG(0, false);
  else if (chunks <= kWave) SMLM_SELECT_BAG(1, false);
  else if (chunks <= 2 * kWave) SMLM_SELECT_BAG(2, false);
  else if (chunks <= 4 * kWave) SMLM_SELECT_BAG(4, false);
  else SMLM_SELECT_BAG(8, false);
#undef SMLM_SELECT_BAG
}

template <bool F32>
void launch_select_bag_table(int table_dtype, const void *s1, const void *s2, int64_t N, int H, int NK, int knn,
                             const void *table, int64_t rows, int D, const uint16_t *scales, const uint16_t *pre,
                             void *out, int out_bf16, void *scores, int64_t *idx, float *w, hipStream_t stream) {
  switch (table_dtype) {
    case SMLM_F32: launch_select_bag<F32, bag::kF32>(s1, s2, N, H, NK, knn, table, rows, D, scales, pre, out, out_bf16, scores, idx, w, stream); break;
    case SMLM_BF16: launch_select_bag<F32, bag::kBF16>(s1, s2, N, H, NK, knn, table, rows, D, scales, pre, out, out_bf16, scores, idx, w, stream); break;
    case SMLM_I8: launch_select_bag<F32, bag::kI8>(s1, s2, N, H, NK, knn, table, rows, D, scales, pre, out, out_bf16, scores, idx, w, stream); break;
    default: launch_select_bag<F32, bag::kQ4>(s1, s2, N, H, NK, knn, table, rows, D, scales, pre, out, out_bf16, scores, idx, w, stream); break;
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
  if (knn < 1 || knn > kMaxKnnGen)
    return fail(SMLM_EUNSUPPORTED, "smlm_pkm_select: knn=%d must be in [1, %d]", knn, kMaxKnnGen);
  if (NK < knn || NK > 65536)
    return fail(SMLM_EUNSUPPORTED, "smlm_pkm_select: NK=%d must be in [knn, 65536]", NK);
  if (N == 0) return SMLM_OK;
  if (dtype == SMLM_F32) launch_select<true>(s1, s2, N * H, NK, knn, scores, idx, w, (hipStream_t)stream);
  else launch_select<false>(s1, s2, N * H, NK, knn, scores, idx, w, (hipStream_t)stream);
  return launch_status("smlm_pkm_select");
}

extern "C" int smlm_pkm_select_bag(const void *s1, const void *s2, int dtype, int64_t N, int H, int NK, int knn,
                                   const void *table, int table_dtype, int64_t rows, int D, const uint16_t *scales,
                                   const uint16_t *pre, void *out, int out_dtype, void *scores, int64_t *idx,
                                   float *w, void *stream) {
  using namespace smlm;
  if (!s1 || !s2 || !table || !out)
    return fail(SMLM_EINVAL, "smlm_pkm_select_bag: null s1, s2, table or out pointer");
  if (dtype != SMLM_BF16 && dtype != SMLM_F32)
    return fail(SMLM_EINVAL, "smlm_pkm_select_bag: dtype must be SMLM_BF16 or SMLM_F32, got %d", dtype);
  if (N < 0 || N > 0x7FFFFFFFLL || H < 1 || H > kFusedMaxHeads)
    return fail(SMLM_EUNSUPPORTED, "smlm_pkm_select_bag: N=%lld, H=%d (1 <= H <= %d)", (long long)N, H,
                kFusedMaxHeads);
  if (knn < 1 || knn > kMaxKnnGen)
    return fail(SMLM_EUNSUPPORTED, "smlm_pkm_select_bag: knn=%d must be in [1, %d]", knn, kMaxKnnGen);
  if (NK < knn || NK > 65536)
    return fail(SMLM_EUNSUPPORTED, "smlm_pkm_select_bag: NK=%d must be in [knn, 65536]", NK);
  if (table_dtype != SMLM_F32 && table_dtype != SMLM_BF16 && table_dtype != SMLM_I8 && table_dtype != SMLM_Q4)
    return fail(SMLM_EINVAL, "smlm_pkm_select_bag: table_dtype %d is not a table format", table_dtype);
  if ((table_dtype == SMLM_I8 || table_dtype == SMLM_Q4) != (scales != nullptr))
    return fail(SMLM_EINVAL, "smlm_pkm_select_bag: scales are required for int8 / q4 tables and only for them");
  if (out_dtype != SMLM_F32 && out_dtype != SMLM_BF16)
    return fail(SMLM_EINVAL, "smlm_pkm_select_bag: out_dtype must be SMLM_F32 or SMLM_BF16");
  const int64_t row_bytes = table_dtype == SMLM_F32 ? 4LL * D : table_dtype == SMLM_BF16 ? 2LL * D
                            : table_dtype == SMLM_I8 ? (int64_t)D : D / 2;
  if (D < 1 || (table_dtype == SMLM_Q4 && D % 2) || row_bytes % 16 || rows < 1 || row_bytes / 16 > 2 * H * kWave)
    return fail(SMLM_EUNSUPPORTED, "smlm_pkm_select_bag: rows of D=%d must be whole 16-byte chunks, at most one per "
                "thread of the %d-thread workgroup", D, 2 * H * kWave);
  if ((uintptr_t)table % 16)
    return fail(SMLM_EINVAL, "smlm_pkm_select_bag: the table must be 16-byte aligned");
  if (N == 0) return SMLM_OK;
  const int out_bf16 = out_dtype == SMLM_BF16;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == SMLM_F32)
    launch_select_bag_table<true>(table_dtype, s1, s2, N, H, NK, knn, table, rows, D, scales, pre, out, out_bf16,
                                  scores, idx, w, s);
  else
    launch_select_bag_table<false>(table_dtype, s1, s2, N, H, NK, knn, table, rows, D, scales, pre, out, out_bf16,
                                   scores, idx, w, s);
  return launch_status("smlm_pkm_select_bag");
}
