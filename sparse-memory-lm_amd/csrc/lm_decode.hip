// Single-token decode attention with a static KV cache: the attention of smlm/model.py:90-107 for one new token
// per sequence (T = 1), fused into one kernel so the captured decode step does not pay ~35 small launches per
// layer.  Per (sequence b, head h), one workgroup:
//   1. RoPE (model.py:63-78: rotate the two halves of the head) on the new token's q and k, in fp32, rounded to
//      bf16 as the bf16 model holds them, by every wavefront for itself through its own LDS row (no workgroup
//      barrier); k and v are written into the cache at the device-side position `pos`;
//   2. scores s_t = q . k_t / sqrt(head_dim) for t = 0..pos, each cache row read with 16-byte loads by
//      head_dim/8 lanes (bf16 pair dot products into fp32: q and k are bf16 values, so the products are exact) and
//      reduced with lane shuffles; the keys and values of a group of passes of rows are in flight together (a
//      decode step is latency-bound), issued after the new token's q, k, v and only for passes that hold rows (raw
//      buffer loads bounded at row pos), so each pass is used as soon as its rows arrive;
//   3. softmax in fp32, by each wavefront over its own rows and in registers: its maximum m_w, the exponentials
//      p_t = exp(s_t - m_w) and their sum l_w (online over the groups of passes: a group that raises the maximum
//      rescales what came before).  Scores are kept in log2 units (s_t log2 e), so each exponential is one exp2;
//   4. the wavefront's y_w = sum_t p_t v_t in registers; then one merge through LDS: m = max m_w,
//      y = sum_w y_w exp(m_w - m) / sum_w l_w exp(m_w - m), written as bf16 into the (B, H*head_dim) layout the
//      output projection reads.
//   (A workgroup-wide softmax would need the scores in LDS and two more barriers and reductions.)
// The PROJ variant folds the output projection (model.py:107, wo) in: y, rounded to bf16 as above, is multiplied by
// the head's column slice of wo, and the n_out fp32 dot products go to parts[b, h, :]; the sum over heads (in head
// order) is left to the consumer (the RMSNORM_PARTS prologue of smlm_decode_linear), one launch fewer per layer.
// The slice's first rows are loaded first of all (they depend on nothing this step computes).
// A position outside [0, min(max_len, rope_len)) writes nothing to the cache and NaN to the output.
#include "pkm_common.h"

namespace smlm {
namespace {

constexpr int kAttnUnroll = 8;    // passes of cache rows whose loads are in flight together

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// v + v[lane ^ MASK] on every lane: quad permutes (1, 2), a row rotation (8) and the gfx950 permlane swaps (16, 32:
// swapping a register with itself leaves v[lane] in one result and v[lane ^ MASK] in the other); other masks
// through ds_bpermute.
template <int MASK>
__device__ __forceinline__ float xor_add(float v) {
  if constexpr (MASK == 1) {
    return v + dpp<0xB1>(v);
  } else if constexpr (MASK == 2) {
    return v + dpp<0x4E>(v);
  } else if constexpr (MASK == 8) {
    return v + dpp<0x128>(v);  // row_ror:8
  } else if constexpr (MASK == 16 || MASK == 32) {
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    const auto pr = MASK == 16 ? __builtin_amdgcn_permlane16_swap(u, u, false, false)
                               : __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return __builtin_bit_cast(float, (uint32_t)pr[0]) + __builtin_bit_cast(float, (uint32_t)pr[1]);
  } else {
    return v + __shfl_xor(v, MASK, kWave);
  }
}

// max(v, v[lane ^ MASK]) on every lane, with the same lane exchanges as xor_add
template <int MASK>
__device__ __forceinline__ float xor_max(float v) {
  if constexpr (MASK == 8) {
    return fmaxf(v, dpp<0x128>(v));  // row_ror:8
  } else if constexpr (MASK == 16 || MASK == 32) {
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    const auto pr = MASK == 16 ? __builtin_amdgcn_permlane16_swap(u, u, false, false)
                               : __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return fmaxf(__builtin_bit_cast(float, (uint32_t)pr[0]), __builtin_bit_cast(float, (uint32_t)pr[1]));
  } else {
    return fmaxf(v, __shfl_xor(v, MASK, kWave));
  }
}

// Maximum over the lanes lane % STRIDE == this lane's (strides 2..32 in doubling steps up to 64).
template <int STRIDE>
__device__ __forceinline__ float strided_max(float v) {
  if constexpr (STRIDE < kWave) {
    v = xor_max<STRIDE>(v);
    return strided_max<STRIDE * 2>(v);
  } else {
    return v;
  }
}

// Sum over aligned groups of G lanes (butterfly: after each step the lanes of a group of 2^k hold its sum, so the
// mirrors of the DPP row act as the xor 4 and xor 8 steps); every lane ends with its group's sum.
template <int G>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (G >= 2) v = xor_add<1>(v);
  if constexpr (G >= 4) v = xor_add<2>(v);
  if constexpr (G >= 8) v += dpp<0x141>(v);   // row_half_mirror
  if constexpr (G >= 16) v += dpp<0x140>(v);  // row_mirror
  if constexpr (G >= 32) v = xor_add<16>(v);
  if constexpr (G >= 64) v = xor_add<32>(v);
  return v;
}

// Sum over the lanes lane % STRIDE == this lane's (strides 2..32 in doubling steps up to 64).
template <int STRIDE>
__device__ __forceinline__ float strided_sum(float v) {
  if constexpr (STRIDE < kWave) {
    v = xor_add<STRIDE>(v);
    return strided_sum<STRIDE * 2>(v);
  } else {
    return v;
  }
}

template <bool ROPE_F32>
__device__ __forceinline__ float table_val(const void *t, int64_t i) {
  if constexpr (ROPE_F32) return ((const float *)t)[i];
  else return bf16_bits_to_f32(((const uint16_t *)t)[i]);
}

__device__ __forceinline__ void unpack8(const uint4 v, float *f) {
  const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    f[2 * e] = __uint_as_float(u[e] << 16);
    f[2 * e + 1] = __uint_as_float(u[e] & 0xFFFF0000u);
  }
}

// Passes of wo rows the projection (PROJ) holds in registers, loaded before the cache rows are used (one pass =
// threads / (head_dim / 8) rows: with 512 threads and head_dim 64, 6 passes = 384 rows, a d_model 384 model's
// whole slice).
template <int kAttnThreads>
constexpr int wo_regs() { return kAttnThreads >= 512 ? 6 : 12; }

template <int N>
struct IntC {
  static constexpr int value = N;
};

// f(IntC<n>{}) for a runtime n in [0, MAX] (a chain of compares): code that needs its count at compile time.
template <int MAX, int N = 0, class F>
__device__ __forceinline__ void with_count(int n, F &&f) {
  if constexpr (N == MAX) {
    f(IntC<N>{});
  } else {
    if (n == N) {
      f(IntC<N>{});
      return;
    }
    with_count<MAX, N + 1>(n, f);
  }
}

// 16-byte loads from a range of n bf16 values through a raw buffer resource (gfx9 layout: base, stride 0,
// num_records in bytes, dword 3 = 0x00020000): a load at or past the end returns zeros and makes no memory access,
// so a wavefront can issue a fixed number of loads whatever the range's length.  Offsets are 32-bit bytes.
struct BufferRows {
  __amdgpu_buffer_rsrc_t r;
  __device__ __forceinline__ BufferRows(const uint16_t *base, int64_t n)
      : r(__builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, (int)(n * 2), 0x00020000)) {}
  __device__ __forceinline__ uint4 load(int elem) const {
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, elem * 2, 0, 0));
  }
};

template <bool ROPE_F32, int HD, int kAttnThreads, bool PROJ>
__global__ void __launch_bounds__(kAttnThreads)
    decode_attention_kernel(const uint16_t *__restrict__ qkv, int64_t qkv_stride, const void *__restrict__ rope_cos,
                            const void *__restrict__ rope_sin, int rope_len, const int64_t *__restrict__ pos_ptr,
                            uint16_t *__restrict__ k_cache, uint16_t *__restrict__ v_cache, int H, int max_len,
                            uint16_t *__restrict__ out, const uint16_t *__restrict__ wo, int64_t wo_stride,
                            int n_out, float *__restrict__ parts) {
  constexpr int kAttnWaves = kAttnThreads / kWave;
  constexpr int LPR = HD / 8;            // lanes per cache row (8 dims, 16 bytes each)
  constexpr int RPW = kWave / LPR;       // rows per wavefront per pass
  constexpr int RPB = RPW * kAttnWaves;  // rows per workgroup per pass
  constexpr int HALF = HD / 2;           // RoPE rotates dim i with dim i + HALF
  constexpr int WR = wo_regs<kAttnThreads>();
  constexpr int RPP = kAttnThreads / LPR;  // wo rows per projection pass (LPR lanes per row, 8 columns each)
  // (the online softmax rescales per group, so the plain and PROJ variants group alike to reach the same y)
  constexpr int U = kAttnUnroll;
  extern __shared__ __align__(16) float smem[];
  float *s_y = smem;                     // [HD] the bf16-rounded output (PROJ)
  float *s_red = s_y + HD;               // [kAttnWaves][HD] the wavefronts' rotated q, later their sums of p * v
  float *s_w = s_red + kAttnWaves * HD;  // [2][kAttnWaves] the wavefronts' maxima, then their sums of p
  float *s_kv = s_w + 2 * kAttnWaves;    // [2][HD] the new token's rotated k and its v (wavefront 0)

  const int b = blockIdx.y, h = blockIdx.x;  // (the grid's linear order is b * H + h)
  const int tid = threadIdx.x, wave = tid / kWave, lane = lane_id();
  const int C = H * HD;
  const uint16_t *row = qkv + (int64_t)b * qkv_stride + h * HD;
  const int64_t cache_row = ((int64_t)b * H + h) * max_len;
  const int sub = lane % LPR, rw = lane / LPR;
  const int slot = wave * RPW + rw;
  const int d0 = sub * 8;  // this lane's 8 dims of the head

  // 0. Loads, in the order they are used (a wavefront's load counter retires in issue order, so anything loaded
  // after the cache rows could only be used once they had all arrived), every one issued on every path so that
  // the counts the compiler waits on are known.  What does not depend on the position is issued before it is read:
  //   the projection's first wo rows (PROJ: row wr0 + i * RPP, columns h * HD + wc * 8 .. + 7, rows past n_out
  //     re-read row n_out - 1);
  //   the new token's q, k and v for the RoPE (lane i: rotation pair i % HALF, 2-byte loads);
  // then, after the position: the pair's rotation factors and, per pass of the first group that holds rows < P, the
  // cache rows (all the keys, then the values; rows at or past P read as zeros without a memory access).  Row P
  // itself is never loaded from the cache.
  const int wc = tid % LPR, wr0 = tid / LPR;
  uint4 wreg[PROJ ? WR : 1];
  if constexpr (PROJ) {
#pragma unroll
    for (int i = 0; i < WR; ++i) {
      const int n = min(wr0 + i * RPP, n_out - 1);
      wreg[i] = *(const uint4 *)(wo + (int64_t)n * wo_stride + h * HD + wc * 8);
    }
  }
  const int pi = lane % HALF;  // this lane's rotation pair
  const uint32_t q1b = row[pi], q2b = row[pi + HALF], k1b = row[C + pi], k2b = row[C + pi + HALF];
  constexpr int HD_HI = HD > kWave ? HD - kWave : 1;  // v dims past the first 64 (head_dim 128)
  const uint32_t vb0 = row[2 * C + lane % HD], vb1 = HD > kWave ? row[2 * C + kWave + lane % HD_HI] : 0;
  // A position outside [0, min(max_len, rope_len)) computes as position 0 (so every address stays in range and no
  // branch holds back the loads above), writes nothing to the cache and NaN to the output.
  const int64_t P_in = *pos_ptr;
  const bool valid = P_in >= 0 && P_in < max_len && P_in < rope_len;
  const int64_t P = valid ? P_in : 0;
  uint16_t *o = PROJ ? nullptr : out + (int64_t)b * C + (int64_t)h * HD;
  float *po = PROJ ? parts + ((int64_t)b * H + h) * n_out : nullptr;
  const float c_rot = table_val<ROPE_F32>(rope_cos, P * HALF + pi);
  const float s_rot = table_val<ROPE_F32>(rope_sin, P * HALF + pi);
  // the cache rows 0..P-1 of (b, h) as raw buffers: a row at or past P reads as zero without a memory access
  const BufferRows krows(k_cache + cache_row * HD, P * HD), vrows(v_cache + cache_row * HD, P * HD);

  const float scale = 1.4426950408889634f * rsqrtf((float)HD);   // log2(e) / sqrt(head_dim): scores in log2 units
  float qf[8];                                   // this lane's 8 dims of the rotated q
  bf16x2 qp[4];                                  // the same as bf16 pairs (exact: q is rounded to bf16)
  float m_run = -INFINITY, l_run = 0.f, acc[8] = {};  // the wavefront's running softmax

  // 1. RoPE (dim i < HALF: x_i c_i - x_{i+HALF} s_i, dim i + HALF: x_i s_i + x_{i+HALF} c_i, in fp32 with one bf16
  // rounding), by every wavefront for itself through its own LDS row (no workgroup barrier); wavefront 0 also
  // writes the new k and v into the cache slot P.  Then row P opens wavefront 0's running softmax (its score, in
  // every lane: the LPR lanes of each row group sum the same dims; its weight and v in row group 0), so the passes
  // cover the cache rows 0..P-1 only.
  auto rope = [&]() {
    const float q1 = bf16_bits_to_f32(q1b), q2 = bf16_bits_to_f32(q2b);
    const float k1 = bf16_bits_to_f32(k1b), k2 = bf16_bits_to_f32(k2b);
    float *s_q = s_red + wave * HD;
    if (lane < HALF) {
      s_q[pi] = round_bf16(q1 * c_rot - q2 * s_rot);
      s_q[pi + HALF] = round_bf16(q1 * s_rot + q2 * c_rot);
    }
    if (wave == 0) {
      const uint32_t ka = bf16_bits_rtne(k1 * c_rot - k2 * s_rot), kb = bf16_bits_rtne(k1 * s_rot + k2 * c_rot);
      if (lane < HALF) {
        s_kv[pi] = bf16_bits_to_f32(ka);
        s_kv[pi + HALF] = bf16_bits_to_f32(kb);
        if (valid) {
          k_cache[(cache_row + P) * HD + pi] = (uint16_t)ka;
          k_cache[(cache_row + P) * HD + pi + HALF] = (uint16_t)kb;
        }
      }
      if (lane < HD) {
        s_kv[HD + lane] = bf16_bits_to_f32(vb0);
        if (valid) v_cache[(cache_row + P) * HD + lane] = (uint16_t)vb0;
      }
      if (HD > kWave && lane < HD - kWave) {
        s_kv[HD + kWave + lane] = bf16_bits_to_f32(vb1);
        if (valid) v_cache[(cache_row + P) * HD + kWave + lane] = (uint16_t)vb1;
      }
    }
    wave_lds_sync();
#pragma unroll
    for (int e = 0; e < 8; ++e) qf[e] = s_q[d0 + e];
#pragma unroll
    for (int e = 0; e < 4; ++e)
      qp[e] = __builtin_bit_cast(bf16x2, (__float_as_uint(qf[2 * e]) >> 16) |
                                             (__float_as_uint(qf[2 * e + 1]) & 0xFFFF0000u));
    if (wave == 0) {
      float dd = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) dd = fmaf(qf[e], s_kv[d0 + e], dd);
      dd = group_sum<LPR>(dd);
      m_run = dd * scale;
      l_run = rw == 0 ? 1.f : 0.f;  // exp(s_P - m_run)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] = rw == 0 ? s_kv[HD + d0 + e] : 0.f;
    }
  };

  // 2-4. Per wavefront, in registers: scores of its rows, their maximum, exponentials and the sum of p * v, over
  // NP passes starting at row t0 with their keys and values in kv, vv (a larger maximum rescales what came before).
  auto passes = [&](const int t0, auto np, const uint4 *kv, const uint4 *vv) {
    constexpr int NP = decltype(np)::value;
    float d[NP > 0 ? NP : 1];
    float gm = -INFINITY;
#pragma unroll
    for (int u = 0; u < NP; ++u) {
      const int t = t0 + u * RPB + slot;
      float dd = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, kv[u].x), qp[0], 0.f, false);
      dd = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, kv[u].y), qp[1], dd, false);
      dd = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, kv[u].z), qp[2], dd, false);
      dd = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, kv[u].w), qp[3], dd, false);
      dd = group_sum<LPR>(dd);
      d[u] = t < P ? dd * scale : -INFINITY;
      gm = fmaxf(gm, d[u]);
    }
    gm = strided_max<LPR>(gm);               // over the wavefront's row groups
    const float m_new = fmaxf(m_run, gm);
    if (m_new == -INFINITY) return;          // wavefront-uniform: none of its rows so far
    const float corr = __builtin_amdgcn_exp2f(m_run - m_new);  // 0 while the wavefront had no row
    l_run *= corr;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] *= corr;
#pragma unroll
    for (int u = 0; u < NP; ++u) {
      const float pt = __builtin_amdgcn_exp2f(d[u] - m_new);  // 0 for rows at or past P
      float vf[8];
      unpack8(vv[u], vf);
      l_run += pt;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] = fmaf(pt, vf[e], acc[e]);
    }
    m_run = m_new;
  };

  // The first group in straight-line code for the number of passes that hold rows < P (each pass then waits only
  // for its own rows, and passes without rows load nothing); later groups (caches longer than RPB * U rows) load
  // their rows after it, in a second round trip.
  const int np0 = (int)min((P + RPB - 1) / RPB, (int64_t)U);
  with_count<U>(np0, [&](auto np) {
    constexpr int NP = decltype(np)::value;
    uint4 kv[NP > 0 ? NP : 1], vv[NP > 0 ? NP : 1];
#pragma unroll
    for (int u = 0; u < NP; ++u) kv[u] = krows.load((u * RPB + slot) * HD + d0);  // keys first: the scores and
#pragma unroll                                                                   // the maximum need every one
    for (int u = 0; u < NP; ++u) vv[u] = vrows.load((u * RPB + slot) * HD + d0);
    // (every load is issued before the arithmetic: otherwise the scheduler may place the RoPE between them, and
    // its waits for q, k, v would hold back the remaining cache rows)
    __builtin_amdgcn_sched_barrier(0);
    rope();
    passes(0, np, kv, vv);
  });
  for (int t0 = RPB * U; t0 < P; t0 += RPB * U) {
    uint4 kv[U], vv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) kv[u] = krows.load((t0 + u * RPB + slot) * HD + d0);
#pragma unroll
    for (int u = 0; u < U; ++u) vv[u] = vrows.load((t0 + u * RPB + slot) * HD + d0);
    passes(t0, IntC<U>{}, kv, vv);
  }
  // the wavefront's row groups summed (lane % LPR keeps the dims; the LPR lanes of a row group hold the same p)
  l_run = strided_sum<LPR>(l_run);
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = strided_sum<LPR>(acc[e]);
  if (rw == 0) {
#pragma unroll
    for (int e = 0; e < 8; ++e) s_red[wave * HD + sub * 8 + e] = acc[e];
  }
  if (lane == 0) {
    s_w[wave] = m_run;
    s_w[kAttnWaves + wave] = l_run;
  }
  __syncthreads();
  // merge: the wavefronts' statistics relative to the largest maximum (row P always counts, so it is finite)
  float mx = s_w[0];
#pragma unroll
  for (int w = 1; w < kAttnWaves; ++w) mx = fmaxf(mx, s_w[w]);
  float fw[kAttnWaves];
  float sum = 0.f;
#pragma unroll
  for (int w = 0; w < kAttnWaves; ++w) {
    fw[w] = __builtin_amdgcn_exp2f(s_w[w] - mx);  // 0 for a wavefront without rows (maximum -inf)
    sum += s_w[kAttnWaves + w] * fw[w];
  }
  const float inv = 1.0f / sum;
  if constexpr (!PROJ) {
    for (int i = tid; i < HD; i += kAttnThreads) {
      float y = 0.f;
#pragma unroll
      for (int w = 0; w < kAttnWaves; ++w) y = fmaf(s_red[w * HD + i], fw[w], y);
      o[i] = valid ? (uint16_t)bf16_bits_rtne(y * inv) : (uint16_t)0x7FC0;  // (bf16 NaN)
    }
  } else {
    // 5. parts[b, h, n] = sum_d bf16(y_d) wo[n, h * HD + d]: LPR lanes per wo row, 8 columns each, reduced with
    // lane shuffles.  y goes through LDS.
    for (int i = tid; i < HD; i += kAttnThreads) {
      float y = 0.f;
#pragma unroll
      for (int w = 0; w < kAttnWaves; ++w) y = fmaf(s_red[w * HD + i], fw[w], y);
      s_y[i] = round_bf16(y * inv);
    }
    __syncthreads();
    bf16x2 yp[4];  // this lane's 8 columns of bf16(y) as bf16 pairs (exact), for pair dot products with wo
#pragma unroll
    for (int e = 0; e < 4; ++e)
      yp[e] = __builtin_bit_cast(bf16x2, (__float_as_uint(s_y[wc * 8 + 2 * e]) >> 16) |
                                             (__float_as_uint(s_y[wc * 8 + 2 * e + 1]) & 0xFFFF0000u));
    for (int base = 0; base < n_out; base += WR * RPP) {
      if (base > 0) {
#pragma unroll
        for (int i = 0; i < WR; ++i) {
          if (base + i * RPP >= n_out) break;  // workgroup-uniform
          const int n = min(base + wr0 + i * RPP, n_out - 1);
          wreg[i] = *(const uint4 *)(wo + (int64_t)n * wo_stride + h * HD + wc * 8);
        }
      }
#pragma unroll
      for (int i = 0; i < WR; ++i) {
        if (base + i * RPP >= n_out) break;  // workgroup-uniform
        float d = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, wreg[i].x), yp[0], 0.f, false);
        d = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, wreg[i].y), yp[1], d, false);
        d = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, wreg[i].z), yp[2], d, false);
        d = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, wreg[i].w), yp[3], d, false);
        d = group_sum<LPR>(d);
        const int n = base + wr0 + i * RPP;
        if (wc == 0 && n < n_out) po[n] = valid ? d : __builtin_nanf("");
      }
    }
  }
}

// Launch arguments of the attention kernels (PROJ: wo and parts set, out unused).
struct AttnArgs {
  const void *qkv;
  int64_t qkv_stride;
  const void *cos, *sin;
  int rope_f32, rope_len;
  const int64_t *pos;
  void *k_cache, *v_cache;
  int64_t B;
  int H, max_len;
  void *out;
  const void *wo;
  int64_t wo_stride;
  int n_out;
  float *parts;
};

template <int HD, int NT, bool PROJ>
int launch_attention_nt(const AttnArgs &a, hipStream_t stream) {
  const size_t shmem = sizeof(float) * (3 * HD + (NT / kWave) * HD + 2 * (NT / kWave));
  const dim3 grid((unsigned)a.H, (unsigned)a.B);
  if (a.rope_f32)
    hipLaunchKernelGGL((decode_attention_kernel<true, HD, NT, PROJ>), grid, dim3(NT), shmem, stream,
                       (const uint16_t *)a.qkv, a.qkv_stride, a.cos, a.sin, a.rope_len, a.pos, (uint16_t *)a.k_cache,
                       (uint16_t *)a.v_cache, a.H, a.max_len, (uint16_t *)a.out, (const uint16_t *)a.wo, a.wo_stride,
                       a.n_out, a.parts);
  else
    hipLaunchKernelGGL((decode_attention_kernel<false, HD, NT, PROJ>), grid, dim3(NT), shmem, stream,
                       (const uint16_t *)a.qkv, a.qkv_stride, a.cos, a.sin, a.rope_len, a.pos, (uint16_t *)a.k_cache,
                       (uint16_t *)a.v_cache, a.H, a.max_len, (uint16_t *)a.out, (const uint16_t *)a.wo, a.wo_stride,
                       a.n_out, a.parts);
  return launch_status("smlm_decode_attention");
}

// 256 threads per (sequence, head) when those workgroups fill the chip twice over, 384 when they fill it once
// (batch 64 x 6 heads: 177.4 -> 176.6 us per decode step against 512; 512 had measured 0.212 -> 0.206 ms against
// 256 there), 512 below that.  The plain and wo-folded variants pick alike, so they reach the same y.  Small batches ran 1024 threads per head until the
// per-wavefront work (its own RoPE, the row-group sums before the merge) outweighed the per-pass arithmetic: with 16
// wavefronts the CU's SIMDs each ran four of those fixed costs; 512 threads measured 127.6 -> 126.6 us per step at
// batch 1 and 135.8 -> 134.0 / 139.6 -> 138.2 / 156.3 -> 155.6 us at batches 8 / 16 / 32 (256: 130.2 at batch 1).
template <int HD, bool PROJ>
int launch_attention(const AttnArgs &a, hipStream_t stream) {
  if (a.B * a.H >= 512) return launch_attention_nt<HD, 256, PROJ>(a, stream);
  if (a.B * a.H >= 256) return launch_attention_nt<HD, 384, PROJ>(a, stream);
  return launch_attention_nt<HD, 512, PROJ>(a, stream);
}

template <bool PROJ>
int launch_attention_hd(const AttnArgs &a, int head_dim, hipStream_t stream) {
  switch (head_dim) {
    case 16: return launch_attention<16, PROJ>(a, stream);
    case 32: return launch_attention<32, PROJ>(a, stream);
    case 64: return launch_attention<64, PROJ>(a, stream);
    case 128: return launch_attention<128, PROJ>(a, stream);
    default: return fail(SMLM_EUNSUPPORTED, "smlm_decode_attention: head_dim %d not in {16, 32, 64, 128}", head_dim);
  }
}

int check_attention(const void *qkv, int64_t qkv_row_stride, const void *rope_cos, const void *rope_sin,
                    int rope_dtype, int rope_len, const int64_t *pos, void *k_cache, void *v_cache, int64_t B, int H,
                    int max_len) {
  if (!qkv || !rope_cos || !rope_sin || !pos || !k_cache || !v_cache)
    return fail(SMLM_EINVAL, "smlm_decode_attention: null pointer argument");
  if (rope_dtype != SMLM_F32 && rope_dtype != SMLM_BF16)
    return fail(SMLM_EINVAL, "smlm_decode_attention: rope tables must be SMLM_F32 or SMLM_BF16");
  if (B < 0 || H < 1 || max_len < 1 || rope_len < 1 || B * (int64_t)H > 0x7FFFFFFFLL)
    return fail(SMLM_EINVAL, "smlm_decode_attention: bad shape B=%lld H=%d max_len=%d", (long long)B, H, max_len);
  if (((int64_t)max_len + 1024) * 128 * 2 > 0x7FFFFFFFLL)  // a (sequence, head)'s rows: 32-bit byte offsets
    return fail(SMLM_EUNSUPPORTED, "smlm_decode_attention: max_len %d too long", max_len);
  if (B > 65535 || H > 65535)  // the grid is (H, B)
    return fail(SMLM_EUNSUPPORTED, "smlm_decode_attention: B=%lld sequences or H=%d heads above 65535",
                (long long)B, H);
  if ((((uintptr_t)qkv | (uintptr_t)k_cache | (uintptr_t)v_cache | (uintptr_t)rope_cos | (uintptr_t)rope_sin) % 16) ||
      qkv_row_stride % 8)
    return fail(SMLM_EINVAL, "smlm_decode_attention: qkv, caches and rope tables must be 16-byte aligned");
  return SMLM_OK;
}

}  // namespace
}  // namespace smlm

extern "C" int smlm_decode_attention(const void *qkv, int64_t qkv_row_stride, const void *rope_cos,
                                     const void *rope_sin, int rope_dtype, int rope_len, const int64_t *pos,
                                     void *k_cache, void *v_cache, int64_t B, int H, int head_dim, int max_len,
                                     void *out, void *stream) {
  using namespace smlm;
  if (!out) return fail(SMLM_EINVAL, "smlm_decode_attention: null pointer argument");
  int rc = check_attention(qkv, qkv_row_stride, rope_cos, rope_sin, rope_dtype, rope_len, pos, k_cache, v_cache, B,
                           H, max_len);
  if (rc != SMLM_OK) return rc;
  if (qkv_row_stride < 3LL * H * head_dim)
    return fail(SMLM_EINVAL, "smlm_decode_attention: qkv_row_stride %lld < 3*H*head_dim", (long long)qkv_row_stride);
  if (B == 0) return SMLM_OK;
  const AttnArgs a{qkv, qkv_row_stride, rope_cos, rope_sin, rope_dtype == SMLM_F32, rope_len, pos, k_cache, v_cache,
                   B, H, max_len, out, nullptr, 0, 0, nullptr};
  return launch_attention_hd<false>(a, head_dim, (hipStream_t)stream);
}

extern "C" int smlm_decode_attention_proj(const void *qkv, int64_t qkv_row_stride, const void *rope_cos,
                                          const void *rope_sin, int rope_dtype, int rope_len, const int64_t *pos,
                                          void *k_cache, void *v_cache, int64_t B, int H, int head_dim, int max_len,
                                          const void *wo, int64_t wo_row_stride, int n_out, float *parts,
                                          void *stream) {
  using namespace smlm;
  if (!wo || !parts) return fail(SMLM_EINVAL, "smlm_decode_attention_proj: null wo or parts");
  int rc = check_attention(qkv, qkv_row_stride, rope_cos, rope_sin, rope_dtype, rope_len, pos, k_cache, v_cache, B,
                           H, max_len);
  if (rc != SMLM_OK) return rc;
  if (qkv_row_stride < 3LL * H * head_dim)
    return fail(SMLM_EINVAL, "smlm_decode_attention: qkv_row_stride %lld < 3*H*head_dim", (long long)qkv_row_stride);
  if (n_out < 1 || wo_row_stride < (int64_t)H * head_dim || wo_row_stride % 8 || (uintptr_t)wo % 16 ||
      (uintptr_t)parts % 4)
    return fail(SMLM_EINVAL, "smlm_decode_attention_proj: wo must be 16-byte aligned (n_out=%d rows of stride %lld "
                "in multiples of 8, >= H*head_dim) and parts 4-byte aligned", n_out, (long long)wo_row_stride);
  if (B == 0) return SMLM_OK;
  const AttnArgs a{qkv, qkv_row_stride, rope_cos, rope_sin, rope_dtype == SMLM_F32, rope_len, pos, k_cache, v_cache,
                   B, H, max_len, nullptr, wo, wo_row_stride, n_out, parts};
  return launch_attention_hd<true>(a, head_dim, (hipStream_t)stream);
}

// ---- SwiGLU activation (smlm/model.py:110-118): out = bf16(silu(a)) * b rounded to bf16, a | b = halves of the
// w13 projection.  The two roundings are the ones the bf16 reference makes (F.silu rounds to bf16, then the
// product rounds).  8 outputs per thread with 16-byte loads and stores.
namespace smlm {
namespace {

__global__ void __launch_bounds__(256) swiglu_kernel(const uint16_t *__restrict__ in, int64_t in_stride,
                                                     uint16_t *__restrict__ out, int64_t M, int hidden) {
  const int per_row = hidden / 8;
  const int64_t item = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (item >= M * per_row) return;
  const int64_t m = item / per_row;
  const int c = (int)(item % per_row) * 8;
  const uint4 av = *(const uint4 *)(in + m * in_stride + c);
  const uint4 bv = *(const uint4 *)(in + m * in_stride + hidden + c);
  float a[8], b[8];
  unpack8(av, a);
  unpack8(bv, b);
  uint32_t o[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float s0 = round_bf16(a[2 * e] / (1.0f + expf(-a[2 * e])));
    const float s1 = round_bf16(a[2 * e + 1] / (1.0f + expf(-a[2 * e + 1])));
    o[e] = bf16_bits_rtne(s0 * b[2 * e]) | (bf16_bits_rtne(s1 * b[2 * e + 1]) << 16);
  }
  *(uint4 *)(out + m * hidden + c) = uint4{o[0], o[1], o[2], o[3]};
}

// ---- greedy step (smlm/train.py:297-299: nxt = logits[:, -1:].argmax(-1)): per row the first index of the
// largest logit; the token is written to tok[b] and to hist[b, pos + 1] (pos read on the device).  1024 threads
// per row, 16-byte loads; keys (order code << 32 | ~index) make "largest value, then lowest index" one max.
constexpr int kArgmaxThreads = 1024;

__device__ __forceinline__ uint64_t argmax_key(uint32_t bits, int i) {
  return ((uint64_t)order16(bits) << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)i);
}

__global__ void __launch_bounds__(kArgmaxThreads)
    argmax_kernel(const uint16_t *__restrict__ logits, int64_t row_stride, int V, const int64_t *__restrict__ pos,
                  int64_t *__restrict__ tok, int64_t *__restrict__ hist, int64_t hist_stride, int64_t hist_len,
                  int vec) {
  __shared__ uint64_t s_best[kArgmaxThreads / kWave];
  const int b = blockIdx.x;
  const uint16_t *row = logits + (int64_t)b * row_stride;
  uint64_t best = 0;
  if (vec) {  // row 16-byte aligned, V % 8 == 0
    for (int c = threadIdx.x; c < V / 8; c += kArgmaxThreads) {
      const uint4 v = *(const uint4 *)(row + c * 8);
      const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint64_t k0 = argmax_key(u[e] & 0xFFFFu, c * 8 + 2 * e);
        const uint64_t k1 = argmax_key(u[e] >> 16, c * 8 + 2 * e + 1);
        best = k0 > best ? k0 : best;
        best = k1 > best ? k1 : best;
      }
    }
  } else {
    for (int i = threadIdx.x; i < V; i += kArgmaxThreads) {
      const uint64_t k = argmax_key(row[i], i);
      best = k > best ? k : best;
    }
  }
  for (int o = kWave / 2; o > 0; o >>= 1) {
    const uint64_t other = __shfl_xor(best, o, kWave);
    best = other > best ? other : best;
  }
  if (lane_id() == 0) s_best[threadIdx.x / kWave] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    best = s_best[0];
    for (int w = 1; w < kArgmaxThreads / kWave; ++w) best = s_best[w] > best ? s_best[w] : best;
    const int64_t t = (int64_t)(0xFFFFFFFFu - (uint32_t)best);
    tok[b] = t;
    if (hist) {
      const int64_t slot = *pos + 1;
      if (slot >= 0 && slot < hist_len) hist[(int64_t)b * hist_stride + slot] = t;
    }
  }
}

// ---- residual add + RMSNorm (smlm/model.py:124-126, 156-163: x = x + sublayer(...); h = norm(x)): one wavefront
// per row writes x + delta (bf16, the residual stream) and RMSNorm of it (fp32 statistics, bf16 out), so the add
// and the next sublayer's norm are one launch.
__global__ void __launch_bounds__(256) add_rmsnorm_kernel(const uint16_t *__restrict__ x,
                                                          const uint16_t *__restrict__ delta,
                                                          const uint16_t *__restrict__ weight, float eps, int64_t M,
                                                          int C, uint16_t *__restrict__ x_out,
                                                          uint16_t *__restrict__ h_out) {
  const int64_t m = (int64_t)blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave;
  if (m >= M) return;
  const int lane = lane_id();
  const uint16_t *xr = x + m * C;
  const uint16_t *dr = delta ? delta + m * C : nullptr;
  float ss = 0.f;
  for (int c = lane; c < C; c += kWave) {
    float v = bf16_bits_to_f32(xr[c]);
    if (dr) v = round_bf16(v + bf16_bits_to_f32(dr[c]));
    ss = fmaf(v, v, ss);
  }
  ss = wave_sum(ss);
  const float rstd = rsqrtf(ss / (float)C + eps);
  for (int c = lane; c < C; c += kWave) {
    float v = bf16_bits_to_f32(xr[c]);
    if (dr) {
      v = round_bf16(v + bf16_bits_to_f32(dr[c]));
      x_out[m * C + c] = (uint16_t)bf16_bits_rtne(v);
    }
    h_out[m * C + c] = (uint16_t)bf16_bits_rtne(v * rstd * bf16_bits_to_f32(weight[c]));
  }
}

// The same with 16 lanes per row and 16-byte accesses, the row held in registers between the statistics and the
// output (C % 8 == 0, C <= 128 * CPQ): 16 rows per workgroup of 256 threads.  Rows past M repeat the last row's
// loads (every lane takes part in the row sums) and store nothing.
__device__ __forceinline__ float row16_add(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false));
  return v;
}

__device__ __forceinline__ uint4 pack8_rtne(const float *f) {
  uint32_t u[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) u[e] = bf16_bits_rtne(f[2 * e]) | (bf16_bits_rtne(f[2 * e + 1]) << 16);
  return uint4{u[0], u[1], u[2], u[3]};
}

template <int CPQ>
__global__ void __launch_bounds__(256) add_rmsnorm_vec_kernel(const uint16_t *__restrict__ x,
                                                              const uint16_t *__restrict__ delta,
                                                              const uint16_t *__restrict__ weight, float eps,
                                                              int64_t M, int C, uint16_t *__restrict__ x_out,
                                                              uint16_t *__restrict__ h_out) {
  const int sub = threadIdx.x & 15;
  const int64_t m = (int64_t)blockIdx.x * 16 + threadIdx.x / 16;
  const bool live = m < M;
  const int64_t row = (live ? m : M - 1) * C;
  const int CH = C / 8;
  uint4 xv[CPQ], dv[CPQ], gv[CPQ];
#pragma unroll
  for (int j = 0; j < CPQ; ++j) {
    const int c = min(sub + 16 * j, CH - 1);
    xv[j] = *(const uint4 *)(x + row + 8 * c);
    if (delta) dv[j] = *(const uint4 *)(delta + row + 8 * c);
    gv[j] = *(const uint4 *)(weight + 8 * c);
  }
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < CPQ; ++j) {
    float v[8];
    unpack8(xv[j], v);
    if (delta) {
      float d[8];
      unpack8(dv[j], d);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = round_bf16(v[e] + d[e]);
      xv[j] = pack8_rtne(v);
    }
    if (sub + 16 * j < CH) {
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = fmaf(v[e], v[e], ss);
    }
  }
  ss = row16_add(ss);
  const float rstd = rsqrtf(ss / (float)C + eps);
  if (!live) return;
#pragma unroll
  for (int j = 0; j < CPQ; ++j) {
    const int c = sub + 16 * j;
    if (c >= CH) continue;
    if (delta) *(uint4 *)(x_out + row + 8 * c) = xv[j];
    float v[8], w[8];
    unpack8(xv[j], v);
    unpack8(gv[j], w);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = v[e] * rstd * w[e];
    *(uint4 *)(h_out + row + 8 * c) = pack8_rtne(v);
  }
}

// ---- eval BatchNorm of the memory query on bf16 rows (smlm/pkm.py:188-191 with running statistics): out[m, c] =
// bf16(x[m, c] * scale[c] + shift[c]), fp32 arithmetic, one pass (no fp32 intermediate tensor).  8 columns per
// thread with 16-byte accesses.
__global__ void __launch_bounds__(256) affine_bf16_kernel(const uint16_t *__restrict__ x, int64_t x_stride,
                                                          const float *__restrict__ scale,
                                                          const float *__restrict__ shift, int64_t M, int C,
                                                          uint16_t *__restrict__ out, int64_t out_stride) {
  const int per_row = C / 8;
  const int64_t item = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (item >= M * per_row) return;
  const int64_t m = item / per_row;
  const int c = (int)(item % per_row) * 8;
  float v[8];
  unpack8(*(const uint4 *)(x + m * x_stride + c), v);
  const float4 s0 = *(const float4 *)(scale + c), s1 = *(const float4 *)(scale + c + 4);
  const float4 b0 = *(const float4 *)(shift + c), b1 = *(const float4 *)(shift + c + 4);
  const float sc[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
  const float sh[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = fmaf(v[e], sc[e], sh[e]);
  *(uint4 *)(out + m * out_stride + c) = pack8_rtne(v);
}

}  // namespace
}  // namespace smlm

extern "C" int smlm_affine_bf16(const void *x, int64_t x_row_stride, const float *scale, const float *shift,
                                int64_t M, int C, void *out, int64_t out_row_stride, void *stream) {
  using namespace smlm;
  if (!x || !scale || !shift || !out) return fail(SMLM_EINVAL, "smlm_affine_bf16: null pointer");
  if (M < 0 || C < 8 || C % 8 || x_row_stride < C || out_row_stride < C || x_row_stride % 8 || out_row_stride % 8)
    return fail(SMLM_EINVAL, "smlm_affine_bf16: bad shape M=%lld C=%d (C a multiple of 8, row strides >= C and "
                             "multiples of 8)", (long long)M, C);
  if (((uintptr_t)x | (uintptr_t)scale | (uintptr_t)shift | (uintptr_t)out) % 16)
    return fail(SMLM_EINVAL, "smlm_affine_bf16: pointers must be 16-byte aligned");
  const int64_t items = M * (C / 8);
  if (items == 0) return SMLM_OK;
  if ((items + 255) / 256 > 0x7FFFFFFFLL) return fail(SMLM_EINVAL, "smlm_affine_bf16: M too large");
  hipLaunchKernelGGL(affine_bf16_kernel, dim3((unsigned)((items + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t *)x, x_row_stride, scale, shift, M, C, (uint16_t *)out, out_row_stride);
  return launch_status("smlm_affine_bf16");
}

extern "C" int smlm_swiglu(const void *in, int64_t in_row_stride, void *out, int64_t M, int hidden, void *stream) {
  using namespace smlm;
  if (!in || !out) return fail(SMLM_EINVAL, "smlm_swiglu: null pointer");
  if (M < 0 || hidden < 8 || hidden % 8 || in_row_stride < 2LL * hidden || in_row_stride % 8)
    return fail(SMLM_EINVAL, "smlm_swiglu: bad shape M=%lld hidden=%d stride=%lld", (long long)M, hidden,
                (long long)in_row_stride);
  if ((((uintptr_t)in | (uintptr_t)out) % 16))
    return fail(SMLM_EINVAL, "smlm_swiglu: in and out must be 16-byte aligned");
  const int64_t items = M * (hidden / 8);
  if (items == 0) return SMLM_OK;
  hipLaunchKernelGGL(swiglu_kernel, dim3((unsigned)((items + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t *)in, in_row_stride, (uint16_t *)out, M, hidden);
  return launch_status("smlm_swiglu");
}

extern "C" int smlm_greedy_argmax(const void *logits, int64_t row_stride, int64_t B, int V, const int64_t *pos,
                                  int64_t *tok, int64_t *hist, int64_t hist_row_stride, int64_t hist_len,
                                  void *stream) {
  using namespace smlm;
  if (!logits || !tok || (hist && !pos)) return fail(SMLM_EINVAL, "smlm_greedy_argmax: null pointer");
  if (B < 0 || B > 0x7FFFFFFFLL || V < 1 || row_stride < V)
    return fail(SMLM_EINVAL, "smlm_greedy_argmax: bad shape B=%lld V=%d", (long long)B, V);
  if (B == 0) return SMLM_OK;
  const int vec = (((uintptr_t)logits % 16) == 0 && row_stride % 8 == 0 && V % 8 == 0) ? 1 : 0;
  hipLaunchKernelGGL(argmax_kernel, dim3((unsigned)B), dim3(kArgmaxThreads), 0, (hipStream_t)stream,
                     (const uint16_t *)logits, row_stride, V, pos, tok, hist, hist_row_stride, hist_len, vec);
  return launch_status("smlm_greedy_argmax");
}

extern "C" int smlm_add_rmsnorm(const void *x, const void *delta, const void *weight, float eps, int64_t M, int C,
                                void *x_out, void *h_out, void *stream) {
  using namespace smlm;
  if (!x || !weight || !h_out || (delta && !x_out)) return fail(SMLM_EINVAL, "smlm_add_rmsnorm: null pointer");
  if (M < 0 || C < 1 || !(eps >= 0.f)) return fail(SMLM_EINVAL, "smlm_add_rmsnorm: bad shape or eps");
  if (M == 0) return SMLM_OK;
  const bool vec = C % 8 == 0 && C <= 512 &&
                   ((uintptr_t)x | (uintptr_t)delta | (uintptr_t)weight | (uintptr_t)x_out | (uintptr_t)h_out) % 16 == 0;
  if (vec) {
    const int64_t vblocks = (M + 15) / 16;
    if (vblocks > 0x7FFFFFFFLL) return fail(SMLM_EINVAL, "smlm_add_rmsnorm: M too large");
    const dim3 g((unsigned)vblocks), b(256);
    hipStream_t s = (hipStream_t)stream;
    const uint16_t *xx = (const uint16_t *)x, *dd = (const uint16_t *)delta, *ww = (const uint16_t *)weight;
    uint16_t *xo = (uint16_t *)x_out, *ho = (uint16_t *)h_out;
    const int cpq = (C / 8 + 15) / 16;
    if (cpq == 1) hipLaunchKernelGGL(add_rmsnorm_vec_kernel<1>, g, b, 0, s, xx, dd, ww, eps, M, C, xo, ho);
    else if (cpq == 2) hipLaunchKernelGGL(add_rmsnorm_vec_kernel<2>, g, b, 0, s, xx, dd, ww, eps, M, C, xo, ho);
    else if (cpq == 3) hipLaunchKernelGGL(add_rmsnorm_vec_kernel<3>, g, b, 0, s, xx, dd, ww, eps, M, C, xo, ho);
    else hipLaunchKernelGGL(add_rmsnorm_vec_kernel<4>, g, b, 0, s, xx, dd, ww, eps, M, C, xo, ho);
    return launch_status("smlm_add_rmsnorm");
  }
  const int64_t blocks = (M + 3) / 4;
  if (blocks > 0x7FFFFFFFLL) return fail(SMLM_EINVAL, "smlm_add_rmsnorm: M too large");
  hipLaunchKernelGGL(add_rmsnorm_kernel, dim3((unsigned)blocks), dim3(4 * kWave), 0, (hipStream_t)stream,
                     (const uint16_t *)x, (const uint16_t *)delta, (const uint16_t *)weight, eps, M, C,
                     (uint16_t *)x_out, (uint16_t *)h_out);
  return launch_status("smlm_add_rmsnorm");
}
