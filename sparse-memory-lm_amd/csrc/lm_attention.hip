// Causal attention of a prefill / prompt pass on the matrix cores (flash-style: the (T, S) score matrix never
// leaves the workgroup).  Replaces F.scaled_dot_product_attention(q, k, v, is_causal=True) and its masked form
// for new tokens after a filled cache (smlm/model.py:97-105): query t of T sits at position S - T + t and sees
// keys 0 .. S - T + t; y = softmax(q k^T / sqrt(hd)) v, bf16 in and out, fp32 statistics and accumulation.
//
// One workgroup = 128 queries of one (batch, head), 4 wavefronts x 32 queries; the keys go by in tiles of 64,
// staged in LDS row-major (two buffers up to head_dim 64: one barrier per tile).  Per tile each wavefront computes
// S^T = K Q^T on v_mfma_f32_16x16x32_bf16 with the keys as the M operand and its queries as N, so a lane (r, g)
// holds keys 4g..4g+3 of each 16-key tile for ONE query (r): the online softmax (running max m, rescale of the
// output) is per lane, with the cross-lane max over the four lane groups by permlane swaps, and the sums of the
// probabilities accumulate on the matrix cores (a 1.0 operand times P^T).  Then
// O^T = V^T P^T with P^T straight from the score registers (rounded to bf16): the k slots of a 32-key step are
// keys {4g..4g+3, 16+4g..16+4g+3} in lane group g for both operands, so the lane's own exp-scores ARE its B
// operand, and V^T's A operand is two transposing 8-byte LDS reads (ds_read_b64_tr_b16) of the row-major value
// tile: in each 16-lane group, lane i receives element i % 4 of the 8-byte chunks that lanes i / 4 + 4 j point
// at (j = 0..3), so lane s pointing at value row key0 + s / 4, dims 16 mt + 4 (s % 4) .. +3 hands lane r the
// four keys key0 .. key0 + 3 of dim 16 mt + r.  The output fragment holds d = 4g..4g+3 of query r, the same
// query as the statistics, so the final 1/l is per lane too.
#include <algorithm>

#include "pkm_common.h"

namespace smlm {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef short short4_t __attribute__((ext_vector_type(4)));

// 4 consecutive 16-bit values of one column of a row-major LDS tile, transposed across lanes (see above)
__device__ __forceinline__ uint2 lds_read_tr16(const uint16_t *p) {
  return __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                       (__attribute__((address_space(3))) short4_t *)(p)));
}

constexpr int kFaBM = 128;  // queries per workgroup
constexpr int kFaBN = 64;   // keys per tile



__device__ __forceinline__ float xor_lane_f(float v, int j) {
  const uint32_t u = __float_as_uint(v);
  return __uint_as_float(j == 16 ? xor_lane<16>(u) : xor_lane<32>(u));
}

template <int HD>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(HD <= 64 ? 3 : 2)))
    flash_attn_kernel(const uint16_t *__restrict__ q, int64_t qsb, int64_t qsh, int64_t qst,
                      const uint16_t *__restrict__ k, int64_t ksb, int64_t ksh, int64_t kst,
                      const uint16_t *__restrict__ v, int64_t vsb, int64_t vsh, int64_t vst,
                      uint16_t *__restrict__ y, int64_t ysb, int64_t ysh, int64_t yst, int B, int H, int T, int S,
                      float scale_log2) {
  constexpr int KS = HD / 32;           // k-steps of the score product
  constexpr int MT = HD / 16;           // 16-wide d tiles of the output
  constexpr int CPR = HD / 8;           // 16-byte chunks per key / value row
  constexpr int LPT = kFaBN * CPR / 256;  // chunks per thread per tile (of K, and of V)
  constexpr int RB = CPR * 16;          // bytes per key / value row in LDS
  constexpr int SW = CPR < 8 ? CPR : 8;  // chunk c of row r sits in slot c ^ (r % SW): conflict-free fragment reads
  __shared__ __align__(16) uint16_t sK[2][kFaBN * HD];
  __shared__ __align__(16) uint16_t sV[2][kFaBN * HD];

  const int BH = B * H;
  const int ntq = (T + kFaBM - 1) / kFaBM;
  const int qt = ntq - 1 - (int)(blockIdx.x / BH);  // the longest query tiles first
  const int bh = (int)(blockIdx.x % BH), b = bh / H, h = bh % H;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, r = lane & 15, g = lane >> 4;
  const int offset = S - T;
  const int q0 = qt * kFaBM;
  const int qw = q0 + wave * 32;  // this wavefront's first query
  const uint16_t *qb = q + b * qsb + h * qsh;
  const uint16_t *kb = k + b * ksb + h * ksh;
  const uint16_t *vb = v + b * vsb + h * vsh;

  // this wavefront's queries as B fragments: query qw + 16 j + r, dims 32 s + 8 g .. +7 (zeros past T)
  bf16x8 bq[2][KS];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int t = qw + 16 * j + r;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const uint4 val = *(const uint4 *)(qb + (int64_t)min(t, T - 1) * qst + 32 * s + 8 * g);
      bq[j][s] = __builtin_bit_cast(bf16x8, t < T ? val : uint4{0u, 0u, 0u, 0u});
    }
  }

  // keys this workgroup needs: up to the position of its last query
  const int kv_end = offset + min(T, q0 + kFaBM);
  const int ntk = (kv_end + kFaBN - 1) / kFaBN;
  const bool wave_on = qw < T;
  const int qpos_lo = offset + qw;                 // position of the wavefront's first query
  const int qpos_hi = offset + min(T - 1, qw + 31);  // ... and of its last

  float m[2] = {-__builtin_inff(), -__builtin_inff()};
  // the sums of the probabilities come from the matrix cores: a 1.0 A operand times P^T puts each query's sum of
  // its (bf16) probabilities in every row of the output tile, so no VALU additions or lane reductions are needed
  floatx4 lacc[2] = {floatx4{0.f, 0.f, 0.f, 0.f}, floatx4{0.f, 0.f, 0.f, 0.f}};
  const bf16x8 ones = __builtin_bit_cast(bf16x8, uint4{0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u});
  floatx4 oacc[MT][2];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int j = 0; j < 2; ++j) oacc[mt][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  // tile loads straight into LDS (buffer loads with the LDS bit: lane i of a wavefront's load writes bytes 16 i ..
  // 16 i + 15 of the wavefront's 1 KB piece): LDS chunk id = tid + 256 u is slot id % CPR of row id / CPR, which
  // holds the row's global chunk slot ^ (row % SW).  The buffers end at row S - 1, so the rows of a partial last
  // tile past S read as zeros.
  const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(
      (void *)kb, (short)0, (int)(((int64_t)(S - 1) * kst + HD) * 2), 0x00020000);
  const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(
      (void *)vb, (short)0, (int)(((int64_t)(S - 1) * vst + HD) * 2), 0x00020000);
  auto load_tile = [&](int kv0, int buf) {
#pragma unroll
    for (int u = 0; u < LPT; ++u) {
      const int id = tid + 256 * u, row = id / CPR, c = (id % CPR) ^ (row % SW);
      const int key = kv0 + row;
      const int piece = (256 * u + wave * kWave) * 16;  // this wavefront's 1 KB of the tile
      __builtin_amdgcn_raw_ptr_buffer_load_lds(krs, (__attribute__((address_space(3))) void *)((char *)sK[buf] + piece),
                                               16, (int)((key * kst + 8 * c) * 2), 0, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(vrs, (__attribute__((address_space(3))) void *)((char *)sV[buf] + piece),
                                               16, (int)((key * vst + 8 * c) * 2), 0, 0, 0);
    }
  };
  load_tile(0, 0);
  __builtin_amdgcn_s_waitcnt(0);  // this thread's pieces of tile 0 are in LDS ...
  __syncthreads();                // ... and everyone's

  for (int tk = 0; tk < ntk; ++tk) {
    const int kv0 = tk * kFaBN;
    const int buf = tk & 1;
    if (tk + 1 < ntk) load_tile(kv0 + kFaBN, buf ^ 1);  // into the buffer every wavefront left at the last barrier

    // wavefront-uniform: tiles none of this wavefront's queries reaches are skipped
    if (wave_on && kv0 <= qpos_hi) {
      const bool masked = kv0 + kFaBN - 1 > qpos_lo;

      // S^T tile: sacc[kt][j][i] = q(query qw + 16 j + r) . k(key kv0 + 16 kt + 4 g + i)
      floatx4 sacc[4][2];
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int j = 0; j < 2; ++j) sacc[kt][j] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        bf16x8 a[4];
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
        const int row = 16 * kt + r;
        a[kt] = *(const bf16x8 *)((const char *)sK[buf] + row * RB + (((4 * s + g) ^ (row % SW)) * 16));
      }
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            sacc[kt][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[kt], bq[j][s], sacc[kt][j], 0, 0, 0);
      }

      // online softmax per query (lane), in the log2 domain.  The reference point m of the exponentials is raised
      // (and the output and sum rescaled) only when some query of the wavefront has a tile maximum more than 2^8
      // above it: until then the probabilities exp2(s - m) stay below 256, exact enough in fp32 and bf16, and the
      // rescale, which costs as much as a tile's products, is skipped.  Every query sees key 0 in tile 0, so m is
      // finite from the first tile on.
      float mx[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int qpos = offset + qw + 16 * j + r;
        if (masked) {
#pragma unroll
          for (int kt = 0; kt < 4; ++kt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int key = kv0 + 16 * kt + 4 * g + i;
              if (key > qpos || key >= S) sacc[kt][j][i] = -__builtin_inff();
            }
        }
        float a = fmaxf(fmaxf(sacc[0][j][0], sacc[0][j][1]), fmaxf(sacc[0][j][2], sacc[0][j][3]));
#pragma unroll
        for (int kt = 1; kt < 4; ++kt)
          a = fmaxf(a, fmaxf(fmaxf(sacc[kt][j][0], sacc[kt][j][1]), fmaxf(sacc[kt][j][2], sacc[kt][j][3])));
        a = fmaxf(a, xor_lane_f(a, 16));
        mx[j] = fmaxf(a, xor_lane_f(a, 32)) * scale_log2;
      }
      if (__builtin_amdgcn_ballot_w64(mx[0] > m[0] + 8.f || mx[1] > m[1] + 8.f)) {  // wavefront-uniform
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const float mnew = fmaxf(m[j], mx[j]);
          const float alpha = __builtin_amdgcn_exp2f(m[j] - mnew);
          lacc[j] *= alpha;
          m[j] = mnew;
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) oacc[mt][j] *= alpha;
        }
      }
      bf16x8 bp[2][2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
          for (int i = 0; i < 4; ++i) sacc[kt][j][i] = __builtin_amdgcn_exp2f(sacc[kt][j][i] * scale_log2 - m[j]);
        // P^T as B fragments: 32-key step ks = key tiles 2 ks and 2 ks + 1
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          const floatx4 lo = sacc[2 * ks][j], hi = sacc[2 * ks + 1][j];
          const uint4 pk{pack_bf16x2(lo[0], lo[1]), pack_bf16x2(lo[2], lo[3]), pack_bf16x2(hi[0], hi[1]),
                         pack_bf16x2(hi[2], hi[3])};
          bp[j][ks] = __builtin_bit_cast(bf16x8, pk);
          lacc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, bp[j][ks], lacc[j], 0, 0, 0);
        }
      }

      // O^T += V^T P^T: A fragment of d tile mt = values of d = 16 mt + r at the step's keys (same slot order),
      // keys 32 ks + 4 g .. +3 (lo) and 32 ks + 16 + 4 g .. +3 (hi), by transposing reads (lane r % 4 of each
      // quarter-row group points at row key0 + r / 4, dims 16 mt + 4 (r % 4) .. +3)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const int row = 32 * ks + 4 * g + r / 4, dim = 16 * mt + 4 * (r % 4);
          const char *src = (const char *)sV[buf] + row * RB + (((dim / 8) ^ (row % SW)) * 16) + (dim % 8) * 2;
          const uint2 lo = lds_read_tr16((const uint16_t *)src),
                      hi = lds_read_tr16((const uint16_t *)(src + 16 * RB));  // row + 16: the same swizzle
          const bf16x8 a = __builtin_bit_cast(bf16x8, uint4{lo.x, lo.y, hi.x, hi.y});
#pragma unroll
          for (int j = 0; j < 2; ++j)
            oacc[mt][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bp[j][ks], oacc[mt][j], 0, 0, 0);
        }
    }

    __builtin_amdgcn_s_waitcnt(0);  // this thread's pieces of the next tile are in LDS ...
    __syncthreads();                // ... and everyone's; every wavefront is done with this tile
  }

  // y[query][d]: lane (r, g) holds d = 16 mt + 4 g .. +3 of query qw + 16 j + r
  if (!wave_on) return;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int t = qw + 16 * j + r;
    if (t >= T) continue;
    const float inv = 1.0f / lacc[j][0];
    uint16_t *yr = y + b * ysb + h * ysh + (int64_t)t * yst;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const floatx4 o = oacc[mt][j];
      *(uint2 *)(yr + 16 * mt + 4 * g) = uint2{pack_bf16x2(o[0] * inv, o[1] * inv), pack_bf16x2(o[2] * inv, o[3] * inv)};
    }
  }
}

template <int HD>
int launch_flash(const void *q, const int64_t *qs, const void *k, const int64_t *ks, const void *v, const int64_t *vs,
                 void *y, const int64_t *ys, int B, int H, int T, int S, hipStream_t stream) {
  const int ntq = (T + kFaBM - 1) / kFaBM;
  const float scale_log2 = 1.4426950408889634f / sqrtf((float)HD);
  hipLaunchKernelGGL((flash_attn_kernel<HD>), dim3((unsigned)((int64_t)ntq * B * H)), dim3(256), 0, stream,
                     (const uint16_t *)q, qs[0], qs[1], qs[2], (const uint16_t *)k, ks[0], ks[1], ks[2],
                     (const uint16_t *)v, vs[0], vs[1], vs[2], (uint16_t *)y, ys[0], ys[1], ys[2], B, H, T, S,
                     scale_log2);
  return launch_status("smlm_prefill_attention");
}

// ---- RoPE of a prompt pass: the (B*T, 3*H*hd) qkv projection -> rotated q and k (and v) in the layouts attention
// reads, one pass instead of the chunk / multiply / add / cat ops of smlm/model.py:63-78.  Token t is at position
// pos0 + t; out1 = bf16(x1 c - x2 s), out2 = bf16(x1 s + x2 c) in fp32 with one rounding each (the formula of the
// decode step's attention kernel, so prompt and decode keys come from the same arithmetic).  One thread per 8
// rotation pairs of a (token, head, q | k), or per 8 dims of v.
__device__ __forceinline__ void unpack8f(const uint4 v, float *f) {
  const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    f[2 * e] = __uint_as_float(u[e] << 16);
    f[2 * e + 1] = __uint_as_float(u[e] & 0xFFFF0000u);
  }
}

template <bool ROPE_F32>
__device__ __forceinline__ void load8_table(const void *t, int64_t i, float *f) {
  if constexpr (ROPE_F32) {
    const float4 a = *(const float4 *)((const float *)t + i), b = *(const float4 *)((const float *)t + i + 4);
    f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w; f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
  } else {
    unpack8f(*(const uint4 *)((const uint16_t *)t + i), f);
  }
}

template <bool ROPE_F32, int HD>
__global__ void __launch_bounds__(256)
    rope_qkv_kernel(const uint16_t *__restrict__ qkv, int64_t qkv_stride, const void *__restrict__ rope_cos,
                    const void *__restrict__ rope_sin, int pos0, uint16_t *__restrict__ q_out, int64_t qsb,
                    int64_t qsh, int64_t qst, uint16_t *__restrict__ k_out, int64_t ksb, int64_t ksh, int64_t kst,
                    uint16_t *__restrict__ v_out, int64_t vsb, int64_t vsh, int64_t vst, int B, int T, int H) {
  constexpr int CQ = HD / 16;  // 8-pair chunks of a q or k head
  constexpr int CV = HD / 8;   // 8-dim chunks of a v head
  const int per_head = 2 * CQ + (v_out ? CV : 0);
  const int64_t total = (int64_t)B * T * H * per_head;
  for (int64_t it = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; it < total;
       it += (int64_t)gridDim.x * blockDim.x) {
    int64_t rest = it;
    const int u = (int)(rest % per_head);
    rest /= per_head;
    const int h = (int)(rest % H);
    rest /= H;
    const int t = (int)(rest % T);
    const int b = (int)(rest / T);
    const uint16_t *row = qkv + ((int64_t)b * T + t) * qkv_stride;
    if (u < 2 * CQ) {
      const int part = u / CQ, c = u % CQ;  // part 0: q, 1: k
      const uint16_t *src = row + (int64_t)part * H * HD + h * HD;
      float x1[8], x2[8], cs[8], sn[8];
      unpack8f(*(const uint4 *)(src + 8 * c), x1);
      unpack8f(*(const uint4 *)(src + HD / 2 + 8 * c), x2);
      const int64_t ti = (int64_t)(pos0 + t) * (HD / 2) + 8 * c;
      load8_table<ROPE_F32>(rope_cos, ti, cs);
      load8_table<ROPE_F32>(rope_sin, ti, sn);
      uint32_t o1[4], o2[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int i0 = 2 * e, i1 = 2 * e + 1;
        o1[e] = bf16_bits_rtne(x1[i0] * cs[i0] - x2[i0] * sn[i0]) |
                (bf16_bits_rtne(x1[i1] * cs[i1] - x2[i1] * sn[i1]) << 16);
        o2[e] = bf16_bits_rtne(x1[i0] * sn[i0] + x2[i0] * cs[i0]) |
                (bf16_bits_rtne(x1[i1] * sn[i1] + x2[i1] * cs[i1]) << 16);
      }
      uint16_t *dst = part == 0 ? q_out + b * qsb + h * qsh + (int64_t)t * qst
                                : k_out + b * ksb + h * ksh + (int64_t)t * kst;
      *(uint4 *)(dst + 8 * c) = uint4{o1[0], o1[1], o1[2], o1[3]};
      *(uint4 *)(dst + HD / 2 + 8 * c) = uint4{o2[0], o2[1], o2[2], o2[3]};
    } else {
      const int c = u - 2 * CQ;
      *(uint4 *)(v_out + b * vsb + h * vsh + (int64_t)t * vst + 8 * c) =
          *(const uint4 *)(row + 2LL * H * HD + h * HD + 8 * c);
    }
  }
}

template <int HD>
int launch_rope(const void *qkv, int64_t qkv_stride, const void *cos, const void *sin, int f32, int pos0, void *q,
                const int64_t *qs, void *k, const int64_t *ks, void *v, const int64_t *vs, int B, int T, int H,
                hipStream_t stream) {
  const int64_t per_head = 2 * (HD / 16) + (v ? HD / 8 : 0);
  const int64_t items = (int64_t)B * T * H * per_head;
  const unsigned grid = (unsigned)std::min<int64_t>((items + 255) / 256, 1 << 16);
  const int64_t z3[3] = {0, 0, 0};
  const int64_t *vv = v ? vs : z3;
  if (f32)
    hipLaunchKernelGGL((rope_qkv_kernel<true, HD>), dim3(grid), dim3(256), 0, stream, (const uint16_t *)qkv,
                       qkv_stride, cos, sin, pos0, (uint16_t *)q, qs[0], qs[1], qs[2], (uint16_t *)k, ks[0], ks[1],
                       ks[2], (uint16_t *)v, vv[0], vv[1], vv[2], B, T, H);
  else
    hipLaunchKernelGGL((rope_qkv_kernel<false, HD>), dim3(grid), dim3(256), 0, stream, (const uint16_t *)qkv,
                       qkv_stride, cos, sin, pos0, (uint16_t *)q, qs[0], qs[1], qs[2], (uint16_t *)k, ks[0], ks[1],
                       ks[2], (uint16_t *)v, vv[0], vv[1], vv[2], B, T, H);
  return launch_status("smlm_rope_qkv");
}

}  // namespace
}  // namespace smlm

extern "C" int smlm_rope_qkv(const void *qkv, int64_t qkv_row_stride, const void *rope_cos, const void *rope_sin,
                             int rope_dtype, int rope_len, int pos0, void *q_out, const int64_t *q_strides,
                             void *k_out, const int64_t *k_strides, void *v_out, const int64_t *v_strides, int64_t B,
                             int T, int H, int head_dim, void *stream) {
  using namespace smlm;
  if (!qkv || !rope_cos || !rope_sin || !q_out || !q_strides || !k_out || !k_strides || (v_out && !v_strides))
    return fail(SMLM_EINVAL, "smlm_rope_qkv: null pointer argument");
  if (rope_dtype != SMLM_F32 && rope_dtype != SMLM_BF16)
    return fail(SMLM_EINVAL, "smlm_rope_qkv: rope tables must be SMLM_F32 or SMLM_BF16");
  if (B < 0 || T < 0 || H < 1 || pos0 < 0 || B * (int64_t)T > 0x7FFFFFFFLL)
    return fail(SMLM_EINVAL, "smlm_rope_qkv: bad shape B=%lld T=%d H=%d pos0=%d", (long long)B, T, H, pos0);
  if ((int64_t)pos0 + T > rope_len)
    return fail(SMLM_EINVAL, "smlm_rope_qkv: positions %d..%d are past the rope table (%d rows)", pos0,
                pos0 + T - 1, rope_len);
  if (head_dim != 16 && head_dim != 32 && head_dim != 64 && head_dim != 128)
    return fail(SMLM_EUNSUPPORTED, "smlm_rope_qkv: head_dim %d not in {16, 32, 64, 128}", head_dim);
  if (qkv_row_stride < 3LL * H * head_dim || qkv_row_stride % 8)
    return fail(SMLM_EINVAL, "smlm_rope_qkv: qkv_row_stride %lld must be >= 3*H*head_dim and a multiple of 8",
                (long long)qkv_row_stride);
  const int64_t *st[3] = {q_strides, k_strides, v_out ? v_strides : q_strides};
  for (int a = 0; a < 3; ++a)
    for (int i = 0; i < 3; ++i)
      if (st[a][i] < 0 || st[a][i] % 8)
        return fail(SMLM_EINVAL, "smlm_rope_qkv: output strides must be non-negative multiples of 8 elements");
  if (((uintptr_t)qkv | (uintptr_t)q_out | (uintptr_t)k_out | (uintptr_t)v_out | (uintptr_t)rope_cos |
       (uintptr_t)rope_sin) % 16)
    return fail(SMLM_EINVAL, "smlm_rope_qkv: qkv, the outputs and the rope tables must be 16-byte aligned");
  if (B == 0 || T == 0) return SMLM_OK;
  const int f32 = rope_dtype == SMLM_F32, b = (int)B;
  hipStream_t s = (hipStream_t)stream;
  switch (head_dim) {
    case 16: return launch_rope<16>(qkv, qkv_row_stride, rope_cos, rope_sin, f32, pos0, q_out, q_strides, k_out, k_strides, v_out, v_strides, b, T, H, s);
    case 32: return launch_rope<32>(qkv, qkv_row_stride, rope_cos, rope_sin, f32, pos0, q_out, q_strides, k_out, k_strides, v_out, v_strides, b, T, H, s);
    case 64: return launch_rope<64>(qkv, qkv_row_stride, rope_cos, rope_sin, f32, pos0, q_out, q_strides, k_out, k_strides, v_out, v_strides, b, T, H, s);
    default: return launch_rope<128>(qkv, qkv_row_stride, rope_cos, rope_sin, f32, pos0, q_out, q_strides, k_out, k_strides, v_out, v_strides, b, T, H, s);
  }
}

extern "C" int smlm_prefill_attention(const void *q, const int64_t *q_strides, const void *k, const int64_t *k_strides,
                                      const void *v, const int64_t *v_strides, void *y, const int64_t *y_strides,
                                      int64_t B, int H, int T, int S, int head_dim, void *stream) {
  using namespace smlm;
  if (!q || !k || !v || !y || !q_strides || !k_strides || !v_strides || !y_strides)
    return fail(SMLM_EINVAL, "smlm_prefill_attention: null pointer argument");
  if (B < 0 || H < 1 || T < 0 || S < T || (T > 0 && S < 1))
    return fail(SMLM_EINVAL, "smlm_prefill_attention: bad shape B=%lld H=%d T=%d S=%d", (long long)B, H, T, S);
  if (head_dim != 32 && head_dim != 64 && head_dim != 128)
    return fail(SMLM_EUNSUPPORTED, "smlm_prefill_attention: head_dim %d not in {32, 64, 128}", head_dim);
  const int64_t ntq = ((int64_t)T + kFaBM - 1) / kFaBM;
  if (ntq * B * H > 0x7FFFFFFFLL)
    return fail(SMLM_EINVAL, "smlm_prefill_attention: B*H*ceil(T/128)=%lld workgroups is too many",
                (long long)(ntq * B * H));
  const int64_t *st[4] = {q_strides, k_strides, v_strides, y_strides};
  for (int a = 0; a < 4; ++a)
    for (int i = 0; i < 3; ++i)
      if (st[a][i] < 0 || st[a][i] % (a == 3 ? 4 : 8))
        return fail(SMLM_EINVAL, "smlm_prefill_attention: strides must be non-negative multiples of 8 elements (4 "
                                 "for y); got %lld", (long long)st[a][i]);
  if (((uintptr_t)q | (uintptr_t)k | (uintptr_t)v) % 16 || (uintptr_t)y % 8)
    return fail(SMLM_EINVAL, "smlm_prefill_attention: q, k, v must be 16-byte and y 8-byte aligned");
  // the key / value tiles are read through 32-bit buffer offsets from each (batch, head)'s first row
  const int64_t row_stride = k_strides[2] > v_strides[2] ? k_strides[2] : v_strides[2];
  if (((int64_t)S + kFaBN) * row_stride * 2 + 2 * head_dim > 0x7FFFFFFFLL)
    return fail(SMLM_EUNSUPPORTED, "smlm_prefill_attention: S=%d keys x row stride %lld elements exceed the 2 GB a "
                "(batch, head)'s key or value rows may span", S, (long long)row_stride);
  if (B == 0 || T == 0) return SMLM_OK;
  hipStream_t s = (hipStream_t)stream;
  const int b = (int)B;
  switch (head_dim) {
    case 32: return launch_flash<32>(q, q_strides, k, k_strides, v, v_strides, y, y_strides, b, H, T, S, s);
    case 64: return launch_flash<64>(q, q_strides, k, k_strides, v, v_strides, y, y_strides, b, H, T, S, s);
    default: return launch_flash<128>(q, q_strides, k, k_strides, v, v_strides, y, y_strides, b, H, T, S, s);
  }
}
