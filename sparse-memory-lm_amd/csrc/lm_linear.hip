// Small-M fused linear layers of the single-token decode step: y = h W^T for M token rows (the decode batch) and
// an (N, K) nn.Linear weight W, on the matrix cores (v_mfma_f32_16x16x32_bf16, fp32 accumulation), with the op in
// front of it and the op after it in the same launch (smlm/model.py:110-163, 266-293; smlm/pkm.py:188-191, 213-224):
//
//   prologue  PLAIN          h = x
//             RMSNORM        xs = bf16(x + delta) (delta optional), h = bf16(xs * rsqrt(mean(xs^2) + eps) * g):
//                            the residual add and the RMSNorm of the next sublayer
//             EMBED_RMSNORM  xs = emb[tok[m]] (the token embedding), then as RMSNORM
//             EMBED_ARGMAX   as EMBED_RMSNORM with tok[m] = the greedy choice from the previous step's ARGMAX
//                            partial keys (each row reduced by the 16 lanes that gather its embedding); column
//                            block 0 writes the tokens and their history slot: no separate argmax launch per step
//             RMSNORM_PARTS  as RMSNORM with delta = bf16(sum_q parts[m, q, :]), fp32 parts summed in q order (the
//                            per-head output projections the attention kernel wrote: wo costs no launch)
//                            xs is written once to x_out (the residual stream), by the column block 0.
//   epilogue  STORE          v = bf16(acc + bias); on the first n_affine columns v = bf16(v * scale + shift) (the
//                            eval BatchNorm of the memory query); columns [0, n_split) go to out, [n_split, N) to
//                            out2 (query_proj and swilu_proj of a memory layer are one launch)
//             SWIGLU         out[:, j] = bf16(bf16(silu(a_j)) * b_j) with a_j = bf16(acc_j), b_j = bf16(acc_{H+j}),
//                            H = N / 2 (w13 + the SwiGLU activation)
//             ARGMAX         per token, the largest key (bf16 logit, then lowest column) over the block's 128
//                            columns, to partial[m, block] (lm_head + greedy argmax; no logits are written)
//
// Workgroup = 4 wavefronts, a token group of 16 or 32 rows x one column block.  STORE / SWIGLU: one 16-column tile
// per workgroup (SWIGLU: the 16 a columns and their 16 b columns), the 4 wavefronts split the contraction and their
// partial sums are added in a fixed order through LDS.  ARGMAX: each wavefront owns 2 tiles (32 columns) over the
// whole contraction.  Every result is deterministic.  With several token groups the grid is 1-D and the groups of
// one column block share an XCD (workgroup id % 8), so its weight rows come from one L2.
//
// Latency is what matters at decode sizes, so every global load a lane needs is issued before the first one is
// used: the prologue's input rows first (addresses clamped into range, no per-row branches; a wavefront's loads
// retire in issue order, so the prologue can start once they are in), then the weight fragments of the lane's K
// slice, then the prologue arithmetic, which overlaps the weights' arrival.  EMBED_ARGMAX issues the argmax keys,
// then the weights, then the embedding rows (whose address needs the keys' reduction).  The prologue works on rows
// of 16 lanes (DPP reductions inside a row) and writes the normalised bf16 rows to LDS ([tokens][K + 8]), from which
// the B fragments are read; a PLAIN input is read into registers directly.
//
// MFMA operand mapping (16x16x32, r = lane % 16, g = lane / 16): A = 16 weight rows x 32 k (lane: row r, k group g),
// B = 32 k x 16 tokens (lane: token r, k group g), D: lane holds columns 4g..4g+3 of token r.
#include "pkm_common.h"

namespace smlm {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kLinThreads = 256;
constexpr int kLinWaves = kLinThreads / kWave;
constexpr int kMaxTiles = 2;      // token tiles of 16 per workgroup, at most (ARGMAX over more than 16 rows)
constexpr int kXcds = 8;          // workgroup id % 8 selects the XCD
constexpr int kArgTiles = 2;      // 16-column tiles per wavefront with the ARGMAX epilogue
constexpr int kArgCols = kLinWaves * kArgTiles * 16;   // 128 columns per workgroup
constexpr uint16_t kBf16NaN = 0x7FC0;

__device__ __forceinline__ float silu_bf16(float a) { return round_bf16_hw(a / (1.0f + expf(-a))); }

__device__ __forceinline__ void unpack8(const uint4 v, float *f) {
  const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    f[2 * e] = __uint_as_float(u[e] << 16);
    f[2 * e + 1] = __uint_as_float(u[e] & 0xFFFF0000u);
  }
}

__device__ __forceinline__ uint4 pack8(const float *f) {
  uint32_t u[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) u[e] = pack_bf16x2(f[2 * e], f[2 * e + 1]);
  return uint4{u[0], u[1], u[2], u[3]};
}

// Sum over the 16 lanes of a DPP row (xor 1, xor 2 within quads, then half-row and row mirrors); every lane of the
// row ends with the row's total.  All 64 lanes must be active.
__device__ __forceinline__ float row16_sum(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false));
  return v;
}

// Prologue: the workgroup's rows [0, nrows) normalised into sH (bf16, row stride KP), rows [nrows, pad_rows) zero.
// Row rr = pass * 16 + wave * 4 + quarter is handled by the 16 lanes of one quarter wavefront; lane `sub` of it owns
// the 16-byte chunks sub, sub + 16, ... (CPQ of them, K <= 128 * CPQ).  load_activations issues every load of the
// prologue (before the weight fragments: they are the workgroup's first use), norm_activations does the arithmetic.
template <int CPQ, int MTB>
struct ActIn {
  uint4 xv[MTB][CPQ], dv[MTB][CPQ], gv[CPQ];
  bool bad[MTB];
};

// The greedy token of row m from ARGMAX partial keys (order16(bf16 logit) << 32 | ~column, 0 = no key): the column
// of the row's largest key, found by the 16 lanes of a quarter wavefront (lane `sub` reads the 16-byte key pairs
// sub, sub + 16, ..., a round's loads in flight together, then a 4-step DPP maximum over the 16 lanes).  The same
// maximum over the same keys as argmax_finish_kernel, so the same token.  The first round's loads are issued before
// the weight fragments (TokKeys), the rest (vocabularies past 32,768 columns) when the keys are reduced.
constexpr int kTokLoads = 8;   // key pairs per lane and round: 256 keys (32,768 columns) per round

template <int MTB>
struct TokKeys {
  uint4 v[MTB][kTokLoads];   // the first round of each pass's row
};

__device__ __forceinline__ uint4 key_pairs(const smlm_linear_args &a, int64_t m, int c) {
  const int npairs = (a.tok_blocks + 1) / 2;
  return *(const uint4 *)(a.tok_partial + m * a.tok_partial_stride + 2 * min(c, npairs - 1));
}

template <int MTB>
__device__ __forceinline__ void load_token_keys(const smlm_linear_args &a, int64_t m0, int nrows, int pad_rows,
                                                TokKeys<MTB> &keys) {
  const int wave = threadIdx.x / kWave, lane = lane_id();
  const int quarter = lane >> 4, sub = lane & 15;
#pragma unroll
  for (int p = 0; p < MTB; ++p) {
    if (p > 0 && p >= pad_rows / 16) continue;     // wavefront-uniform (pass 0 always has a row: no branch)
    const int64_t m = m0 + min(p * 16 + wave * 4 + quarter, nrows - 1);
#pragma unroll
    for (int j = 0; j < kTokLoads; ++j) keys.v[p][j] = key_pairs(a, m, sub + 16 * j);
  }
}

template <int CTRL>
__device__ __forceinline__ uint64_t dpp_u64(uint64_t v) {
  const int lo = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)v, CTRL, 0xF, 0xF, false);
  const int hi = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)(v >> 32), CTRL, 0xF, 0xF, false);
  return ((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo;
}

// The largest key of a round of pairs c0 + sub + 16 j (pairs past the row repeat its last pair; a pair's second key
// past tok_blocks is the stride's pad and counts as 0).
__device__ __forceinline__ uint64_t max_of_pairs(const smlm_linear_args &a, const uint4 *v, int c0, int sub,
                                                 uint64_t best) {
  const int nb = a.tok_blocks, npairs = (nb + 1) / 2;
#pragma unroll
  for (int j = 0; j < kTokLoads; ++j) {
    const int c = min(c0 + sub + 16 * j, npairs - 1);
    const uint64_t k0 = ((uint64_t)v[j].y << 32) | v[j].x;
    const uint64_t k1 = 2 * c + 1 < nb ? ((uint64_t)v[j].w << 32) | v[j].z : 0;
    best = max(best, max(k0, k1));
  }
  return best;
}

// All 64 lanes active: every lane ends with the maximum of its 16-lane row (the lane patterns of row16_sum).
__device__ __forceinline__ int64_t row_argmax_token(const smlm_linear_args &a, int64_t m, int sub,
                                                    const uint4 *first) {
  const int npairs = (a.tok_blocks + 1) / 2;
  uint64_t best = max_of_pairs(a, first, 0, sub, 0);
  for (int c0 = 16 * kTokLoads; c0 < npairs; c0 += 16 * kTokLoads) {
    uint4 v[kTokLoads];
#pragma unroll
    for (int j = 0; j < kTokLoads; ++j) v[j] = key_pairs(a, m, c0 + sub + 16 * j);
    best = max_of_pairs(a, v, c0, sub, best);
  }
  best = max(best, dpp_u64<0xB1>(best));
  best = max(best, dpp_u64<0x4E>(best));
  best = max(best, dpp_u64<0x141>(best));
  best = max(best, dpp_u64<0x140>(best));
  return (int64_t)(0xFFFFFFFFu - (uint32_t)best);
}

template <int PRO, int CPQ, int MTB>
__device__ __forceinline__ void load_activations(const smlm_linear_args &a, int64_t m0, int nrows, int pad_rows,
                                                 bool first_block, ActIn<CPQ, MTB> &in,
                                                 const TokKeys<MTB> *keys = nullptr) {
  constexpr bool EMB = PRO == SMLM_LIN_EMBED_RMSNORM || PRO == SMLM_LIN_EMBED_ARGMAX;
  const int K = a.K, CH = K / 8;
  const int wave = threadIdx.x / kWave, lane = lane_id();
  const int quarter = lane >> 4, sub = lane & 15;
  const int passes = pad_rows / 16;
  const uint16_t *nw = (const uint16_t *)a.norm_w;
  auto &xv = in.xv;
  auto &dv = in.dv;
  auto &gv = in.gv;
  auto &bad = in.bad;
  // EMBED_ARGMAX: column block 0 writes each row's token (and history slot *pos, read before anything else)
  const bool writer = PRO == SMLM_LIN_EMBED_ARGMAX && first_block;
  const int64_t hslot = writer && a.hist ? *a.pos : -1;
#pragma unroll
  for (int j = 0; j < CPQ; ++j) gv[j] = *(const uint4 *)(nw + min(sub + 16 * j, CH - 1) * 8);
#pragma unroll
  for (int p = 0; p < MTB; ++p) {
    bad[p] = false;
    if (p >= passes) continue;                      // wavefront-uniform
    const int rr = p * 16 + wave * 4 + quarter;
    const int64_t m = m0 + min(rr, nrows - 1);      // rows past the end re-read the last row (written as zero)
    const uint16_t *src;
    if constexpr (EMB) {
      int64_t t;
      if constexpr (PRO == SMLM_LIN_EMBED_ARGMAX) {
        t = row_argmax_token(a, m, sub, keys->v[p]);
        if (writer && sub == 0 && rr < nrows) {
          if (a.tok_out) a.tok_out[m] = t;
          if (hslot >= 0 && hslot < a.hist_len) a.hist[m * a.hist_stride + hslot] = t;
        }
      } else {
        t = a.tok[m];
      }
      bad[p] = t < 0 || t >= a.emb_rows;
      src = (const uint16_t *)a.emb + (bad[p] ? 0 : t) * (int64_t)K;
    } else {
      src = (const uint16_t *)a.x + m * a.x_stride;
    }
#pragma unroll
    for (int j = 0; j < CPQ; ++j) xv[p][j] = *(const uint4 *)(src + min(sub + 16 * j, CH - 1) * 8);
    if constexpr (PRO == SMLM_LIN_RMSNORM) {
      if (a.delta) {
        const uint16_t *dsrc = (const uint16_t *)a.delta + m * (int64_t)K;
#pragma unroll
        for (int j = 0; j < CPQ; ++j) dv[p][j] = *(const uint4 *)(dsrc + min(sub + 16 * j, CH - 1) * 8);
      }
    }
  }
}

// RMSNORM_PARTS: delta rows from fp32 parts, one row per wavefront (token groups of kPartsRows = 4 rows, row `wave`
// of the group for wavefront `wave`).  load_parts issues the row's loads before the weight fragments: its parts with
// a lane per 8-column chunk (K <= 512), then its x row and the norm weights in the RMSNORM layout (lane `sub` of each
// 16-lane quarter: chunks sub, sub + 16, ...).  parts_norm adds the parts in part order, rounds once to bf16, moves
// the chunks to the RMSNORM layout with lane swaps (chunk sub + 16 j is lane sub ^ 16 j) and finishes the row with
// the arithmetic of norm_activations in the same lanes and order, so the result is the RMSNORM prologue's on that
// bf16 delta bit for bit; every quarter computes the row, the first stores it.  No LDS round trip and no barrier
// between the sum and the norm, and the group's rows are normalised by four wavefronts at once.
constexpr int kMaxParts = 8;
constexpr int kPartsRows = kLinWaves;
// PLAIN prologue (the attention output, FFN down and value projections): 8-row token groups, so that each
// workgroup pulls half the activation rows through its CU
constexpr int kSmallRows = 8;

// token rows per group of a launch (the kernel's TB and the host's grid agree through this one function)
__host__ __device__ constexpr int group_rows(int pro, int epi, int mtb) {
  return pro == SMLM_LIN_RMSNORM_PARTS ? kPartsRows
         : pro == SMLM_LIN_PLAIN && epi == SMLM_LIN_STORE && mtb == 1 ? kSmallRows
         : mtb * 16;
}

template <int CPQ>
struct PartsIn {
  uint4 pv[kMaxParts][2], xv[CPQ], gv[CPQ];
};

template <int CPQ>
__device__ __forceinline__ void load_parts(const smlm_linear_args &a, int64_t m0, int nrows, PartsIn<CPQ> &in) {
  const int CH = a.K / 8, lane = lane_id(), wave = threadIdx.x / kWave, sub = lane & 15;
  if (wave >= nrows) return;  // wavefront-uniform
  const int64_t m = m0 + wave;
  const float *src = (const float *)a.delta + m * (int64_t)a.delta_parts * a.K + min(lane, CH - 1) * 8;
#pragma unroll
  for (int q = 0; q < kMaxParts; ++q) {
    if (q >= a.delta_parts) break;  // uniform
    const float *pq = src + (int64_t)q * a.K;
    in.pv[q][0] = *(const uint4 *)pq;
    in.pv[q][1] = *(const uint4 *)(pq + 4);
  }
  const uint16_t *xs = (const uint16_t *)a.x + m * a.x_stride, *nw = (const uint16_t *)a.norm_w;
#pragma unroll
  for (int j = 0; j < CPQ; ++j) {
    const int c = min(sub + 16 * j, CH - 1);
    in.xv[j] = *(const uint4 *)(xs + c * 8);
    in.gv[j] = *(const uint4 *)(nw + c * 8);
  }
}

template <int J>
__device__ __forceinline__ uint4 xor_lane4(uint4 v) {
  return uint4{xor_lane<J>(v.x), xor_lane<J>(v.y), xor_lane<J>(v.z), xor_lane<J>(v.w)};
}

template <int CPQ>
__device__ __forceinline__ void parts_norm(const smlm_linear_args &a, int64_t m0, int nrows, uint16_t *sH, int KP,
                                           bool first_block, PartsIn<CPQ> &in) {
  static_assert(CPQ <= 4, "parts prologue: K <= 512");
  const int K = a.K, CH = K / 8, lane = lane_id(), wave = threadIdx.x / kWave;
  const int quarter = lane >> 4, sub = lane & 15;
  if (quarter > 0) {  // rows kPartsRows..15 of the 16-row tile are zero: three per wavefront
    uint16_t *z = sH + (kPartsRows + wave * 3 + quarter - 1) * KP;
#pragma unroll
    for (int j = 0; j < CPQ; ++j)
      if (sub + 16 * j < CH) *(uint4 *)(z + (sub + 16 * j) * 8) = uint4{0u, 0u, 0u, 0u};
  }
  uint16_t *dst = sH + wave * KP;
  if (wave >= nrows) {  // wavefront-uniform: a row past the end is zero
#pragma unroll
    for (int j = 0; j < CPQ; ++j)
      if (quarter == 0 && sub + 16 * j < CH) *(uint4 *)(dst + (sub + 16 * j) * 8) = uint4{0u, 0u, 0u, 0u};
    return;
  }
  float acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.f;
#pragma unroll
  for (int q = 0; q < kMaxParts; ++q) {
    if (q >= a.delta_parts) break;
    const uint4 u0 = in.pv[q][0], u1 = in.pv[q][1];
    const uint32_t w[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] += __uint_as_float(w[e]);
  }
  const uint4 dl = pack8(acc);  // this lane's chunk of the bf16 delta row
  uint4 dv[CPQ];
  dv[0] = dl;
  if constexpr (CPQ > 1) dv[1] = xor_lane4<16>(dl);
  if constexpr (CPQ > 2) dv[2] = xor_lane4<32>(dl);
  if constexpr (CPQ > 3) dv[3] = xor_lane4<16>(xor_lane4<32>(dl));
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < CPQ; ++j) {
    float xf[8], df[8];
    unpack8(in.xv[j], xf);
    unpack8(dv[j], df);
#pragma unroll
    for (int e = 0; e < 8; ++e) xf[e] += df[e];
    in.xv[j] = pack8(xf);                           // the residual stream is bf16: round the sum
    unpack8(in.xv[j], xf);
    if (sub + 16 * j < CH) {
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = fmaf(xf[e], xf[e], ss);
    }
  }
  ss = row16_sum(ss);
  const float rstd = rsqrtf(ss / (float)K + a.eps);
  const bool write_x = a.x_out != nullptr && first_block;
#pragma unroll
  for (int j = 0; j < CPQ; ++j) {
    const int c = sub + 16 * j;
    if (quarter != 0 || c >= CH) continue;
    if (write_x) *(uint4 *)((uint16_t *)a.x_out + (m0 + wave) * (int64_t)K + c * 8) = in.xv[j];
    float xf[8], gf[8];
    unpack8(in.xv[j], xf);
    unpack8(in.gv[j], gf);
#pragma unroll
    for (int e = 0; e < 8; ++e) xf[e] = xf[e] * rstd * gf[e];
    *(uint4 *)(dst + c * 8) = pack8(xf);
  }
}

template <int PRO, int CPQ, int MTB>
__device__ __forceinline__ void norm_activations(const smlm_linear_args &a, int64_t m0, int nrows, int pad_rows,
                                                 uint16_t *sH, int KP, bool first_block, ActIn<CPQ, MTB> &in) {
  const int K = a.K, CH = K / 8;
  const int wave = threadIdx.x / kWave, lane = lane_id();
  const int quarter = lane >> 4, sub = lane & 15;
  const int passes = pad_rows / 16;
  const bool write_x = a.x_out != nullptr && first_block;
  auto &xv = in.xv;
  auto &dv = in.dv;
  auto &gv = in.gv;
  auto &bad = in.bad;
#pragma unroll
  for (int p = 0; p < MTB; ++p) {
    if (p >= passes) continue;
    const int rr = p * 16 + wave * 4 + quarter;
    const bool live = rr < nrows;
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < CPQ; ++j) {
      float xf[8];
      unpack8(xv[p][j], xf);
      if constexpr (PRO == SMLM_LIN_RMSNORM) {
        if (a.delta) {
          float df[8];
          unpack8(dv[p][j], df);
#pragma unroll
          for (int e = 0; e < 8; ++e) xf[e] += df[e];
          xv[p][j] = pack8(xf);                     // the residual stream is bf16: round the sum
          unpack8(xv[p][j], xf);
        }
      }
      if (bad[p]) {                                 // token id outside the embedding: a NaN row
        const uint32_t nn = (uint32_t)kBf16NaN | ((uint32_t)kBf16NaN << 16);
        xv[p][j] = uint4{nn, nn, nn, nn};
        unpack8(xv[p][j], xf);
      }
      if (sub + 16 * j < CH) {
#pragma unroll
        for (int e = 0; e < 8; ++e) ss = fmaf(xf[e], xf[e], ss);
      }
    }
    ss = row16_sum(ss);
    const float rstd = rsqrtf(ss / (float)K + a.eps);
    uint16_t *dst = sH + rr * KP;
#pragma unroll
    for (int j = 0; j < CPQ; ++j) {
      const int c = sub + 16 * j;
      if (c >= CH) continue;
      if (!live) {
        *(uint4 *)(dst + c * 8) = uint4{0u, 0u, 0u, 0u};
        continue;
      }
      if (write_x) *(uint4 *)((uint16_t *)a.x_out + (m0 + rr) * (int64_t)K + c * 8) = xv[p][j];
      float xf[8], gf[8];
      unpack8(xv[p][j], xf);
      unpack8(gv[j], gf);
#pragma unroll
      for (int e = 0; e < 8; ++e) xf[e] = xf[e] * rstd * gf[e];
      *(uint4 *)(dst + c * 8) = pack8(xf);
    }
  }
}

// PRO / EPI: prologue and epilogue; MAXS: k-steps of 32 per wavefront held in registers (>= its K slice);
// CPQ: prologue chunks per lane; MTB: token tiles of 16 per workgroup.  ncb column blocks x ntg token groups.
template <int PRO, int EPI, int MAXS, int CPQ, int MTB>
__global__ void __launch_bounds__(kLinThreads) linear_kernel(const smlm_linear_args a, int ncb, int ntg) {
  constexpr bool ARG = EPI == SMLM_LIN_ARGMAX;
  constexpr int KS = ARG ? 1 : kLinWaves;               // wavefronts along the contraction
  constexpr int NT = EPI == SMLM_LIN_STORE ? 1 : 2;     // weight tiles per wavefront
  extern __shared__ __align__(16) unsigned char smem[];
  const int K = a.K, KP = K + 8;
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  const int r = lane & 15, g = lane >> 4;
  constexpr int TB = group_rows(PRO, EPI, MTB);  // token rows per group
  int cb = (int)blockIdx.x, tg = 0;
  if (ntg > 1) {  // id = ((cb / 8) * ntg + tg) * 8 + cb % 8: the token groups of a column block on one XCD
    const int q = (int)blockIdx.x / kXcds;
    cb = q / ntg * kXcds + (int)blockIdx.x % kXcds;
    tg = q % ntg;
    if (cb >= ncb) return;                          // padding of the last XCD round: the whole workgroup leaves
  }
  const int64_t m0 = (int64_t)tg * TB;
  const int nrows = (int)min((int64_t)TB, a.M - m0);
  const int MT = (nrows + 15) / 16;
  uint16_t *sH = (uint16_t *)smem;

  // this wavefront's K slice [s_lo, s_lo + ns) in steps of 32, and its weight rows
  const int ks = ARG ? 0 : wave;
  const int nsteps = K / 32;
  const int s_lo = ks * nsteps / KS, ns = (ks + 1) * nsteps / KS - s_lo;
  const int cols = EPI == SMLM_LIN_SWIGLU ? a.N / 2 : a.N;                   // output columns
  const int col0 = ARG ? cb * kArgCols + wave * kArgTiles * 16 : cb * 16;
  const uint16_t *W = (const uint16_t *)a.w;

  // STORE epilogue parameters (bias, affine scale / shift) of wavefront 0's 4 columns, loaded before everything
  // else: read in the epilogue they would add a memory round trip of their own after the products
  float ep_bias[4] = {0.f, 0.f, 0.f, 0.f}, ep_sc[4] = {1.f, 1.f, 1.f, 1.f}, ep_sh[4] = {0.f, 0.f, 0.f, 0.f};
  if constexpr (EPI == SMLM_LIN_STORE) {
    const int c = col0 + 4 * g;
    if (ks == 0 && c < cols) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (a.bias) ep_bias[e] = bf16_bits_to_f32(((const uint16_t *)a.bias)[c + e]);
        if (c < a.n_affine) {
          ep_sc[e] = a.scale[c + e];
          ep_sh[e] = a.shift[c + e];
        }
      }
    }
  }

  // 1. the prologue's loads, then the weight fragments (rows past N and steps past the slice re-read valid memory;
  // their products are unused): the prologue's arithmetic then overlaps the weights' arrival
  ActIn<CPQ, PRO == SMLM_LIN_PLAIN ? 1 : MTB> act;
  // ARGMAX with pos_advance: the first workgroup reads the position now and writes it + 1 at its end
  const bool advance = ARG && a.pos_advance != nullptr && blockIdx.x == 0;
  const int64_t pos_now = advance ? *a.pos_advance : 0;
  // EMBED_ARGMAX: the keys, then the weight fragments (in flight during the keys' reduction and the embedding rows'
  // round trip), then the rows
  TokKeys<PRO == SMLM_LIN_EMBED_ARGMAX ? MTB : 1> keys;
  if constexpr (PRO == SMLM_LIN_EMBED_ARGMAX) load_token_keys<MTB>(a, m0, nrows, MT * 16, keys);
  if constexpr (PRO != SMLM_LIN_PLAIN && PRO != SMLM_LIN_RMSNORM_PARTS && PRO != SMLM_LIN_EMBED_ARGMAX)
    load_activations<PRO, CPQ, MTB>(a, m0, nrows, MT * 16, cb == 0, act);
  PartsIn<CPQ> parts_in;
  if constexpr (PRO == SMLM_LIN_RMSNORM_PARTS) load_parts<CPQ>(a, m0, nrows, parts_in);
  uint4 areg[NT][MAXS];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    int wrow = EPI == SMLM_LIN_SWIGLU ? (t == 0 ? col0 : cols + col0) + r : col0 + t * 16 + r;
    wrow = min(wrow, a.N - 1);
    const uint16_t *wp = W + (int64_t)wrow * K + g * 8;
#pragma unroll
    for (int s = 0; s < MAXS; ++s) {
      const int step = min(s_lo + min(s, ns - 1), nsteps - 1);
      areg[t][s] = *(const uint4 *)(wp + max(step, 0) * 32);
    }
  }
  if constexpr (PRO == SMLM_LIN_EMBED_ARGMAX) {
    __builtin_amdgcn_sched_barrier(0);   // the keys' reduction stays behind the weight loads
    load_activations<PRO, CPQ, MTB>(a, m0, nrows, MT * 16, cb == 0, act, &keys);
  }

  // 2. activations: PLAIN rows straight into registers; otherwise the prologue into LDS
  uint4 breg[MTB][PRO == SMLM_LIN_PLAIN ? MAXS : 1];
  if constexpr (PRO == SMLM_LIN_PLAIN) {
#pragma unroll
    for (int mt = 0; mt < MTB; ++mt) {
      if (mt >= MT) continue;                       // wavefront-uniform
      const int tok = min(mt * 16 + r, nrows - 1);
      const uint16_t *xp = (const uint16_t *)a.x + (m0 + tok) * a.x_stride + g * 8;
#pragma unroll
      for (int s = 0; s < MAXS; ++s) {
        const int step = min(s_lo + min(s, ns - 1), nsteps - 1);
        breg[mt][s] = *(const uint4 *)(xp + max(step, 0) * 32);
      }
    }
  } else {
    if constexpr (PRO == SMLM_LIN_RMSNORM_PARTS) parts_norm<CPQ>(a, m0, nrows, sH, KP, cb == 0, parts_in);
    else norm_activations<PRO, CPQ, MTB>(a, m0, nrows, MT * 16, sH, KP, cb == 0, act);
    __syncthreads();
  }

  // 3. products
  floatx4 acc[NT][MTB];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int mt = 0; mt < MTB; ++mt) acc[t][mt] = floatx4{0.f, 0.f, 0.f, 0.f};
  if (MT == MTB && ns == MAXS) {                    // every tile and step present: straight-line code
#pragma unroll
    for (int s = 0; s < MAXS; ++s) {
      const int k = (s_lo + s) * 32 + g * 8;
#pragma unroll
      for (int mt = 0; mt < MTB; ++mt) {
        uint4 b;
        if constexpr (PRO == SMLM_LIN_PLAIN) b = breg[mt][s];
        else b = *(const uint4 *)(sH + (mt * 16 + r) * KP + k);
#pragma unroll
        for (int t = 0; t < NT; ++t)
          acc[t][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, areg[t][s]),
                                                               __builtin_bit_cast(bf16x8, b), acc[t][mt], 0, 0, 0);
      }
    }
  } else {
#pragma unroll
    for (int s = 0; s < MAXS; ++s) {
      if (s >= ns) continue;                          // wavefront-uniform
      const int k = (s_lo + s) * 32 + g * 8;
#pragma unroll
      for (int mt = 0; mt < MTB; ++mt) {
        if (mt >= MT) continue;
        uint4 b;
        if constexpr (PRO == SMLM_LIN_PLAIN) b = breg[mt][s];
        else b = *(const uint4 *)(sH + (mt * 16 + r) * KP + k);
#pragma unroll
        for (int t = 0; t < NT; ++t)
          acc[t][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, areg[t][s]),
                                                               __builtin_bit_cast(bf16x8, b), acc[t][mt], 0, 0, 0);
      }
    }
  }

  if constexpr (KS > 1) {
    // partial sums of wavefronts 1..3 into LDS (over the activations, which every wavefront has finished reading
    // after the barrier), added by wavefront 0 in order
    floatx4 *sRed = (floatx4 *)smem;
    if constexpr (PRO != SMLM_LIN_PLAIN) __syncthreads();
    if (ks > 0) {
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int mt = 0; mt < MTB; ++mt)
          if (mt < MT) sRed[(((ks - 1) * NT + t) * MTB + mt) * kWave + lane] = acc[t][mt];
    }
    __syncthreads();
    if (ks > 0) return;
#pragma unroll
    for (int k2 = 1; k2 < KS; ++k2)
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int mt = 0; mt < MTB; ++mt)
          if (mt < MT) acc[t][mt] += sRed[(((k2 - 1) * NT + t) * MTB + mt) * kWave + lane];
  }

  const int c = col0 + 4 * g;  // this lane's 4 columns c .. c+3 of tile 0 (cols % 16 == 0: all in or all out)
  if constexpr (EPI == SMLM_LIN_STORE) {
    if (c >= cols) return;
    const bool affine = c < a.n_affine;
    const bool first = c < a.n_split;
    uint16_t *dst = first ? (uint16_t *)a.out + c : (uint16_t *)a.out2 + (c - a.n_split);
    const int64_t stride = first ? a.out_stride : a.out2_stride;
#pragma unroll
    for (int mt = 0; mt < MTB; ++mt) {
      const int tok = mt * 16 + r;
      if (mt >= MT || tok >= nrows) continue;
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[e] = acc[0][mt][e] + ep_bias[e];
        if (affine) v[e] = fmaf(round_bf16_hw(v[e]), ep_sc[e], ep_sh[e]);
      }
      *(uint2 *)(dst + (m0 + tok) * stride) = uint2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
    }
  } else if constexpr (EPI == SMLM_LIN_SWIGLU) {
    if (c >= cols) return;
#pragma unroll
    for (int mt = 0; mt < MTB; ++mt) {
      const int tok = mt * 16 + r;
      if (mt >= MT || tok >= nrows) continue;
      float o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = silu_bf16(round_bf16_hw(acc[0][mt][e])) * round_bf16_hw(acc[1][mt][e]);
      *(uint2 *)((uint16_t *)a.out + (m0 + tok) * a.out_stride + c) = uint2{pack_bf16x2(o[0], o[1]),
                                                                            pack_bf16x2(o[2], o[3])};
    }
  } else {  // ARGMAX
    // 32-bit keys inside the workgroup (order16(bf16 logit) << 16 | 0xFFFF - column in the block), maxima over the
    // lane groups by permlane swaps, over the wavefronts through LDS; the partial is the 64-bit key of the result
    uint32_t *sArg = (uint32_t *)smem;  // [4 wavefronts][TB tokens]
    if constexpr (PRO != SMLM_LIN_PLAIN) __syncthreads();  // activations no longer read
#pragma unroll
    for (int mt = 0; mt < MTB; ++mt) {
      if (mt >= MT) continue;
      uint32_t best = 0;
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int local = wave * kArgTiles * 16 + 4 * g + t * 16 + e;   // column - cb * kArgCols
          if (c + t * 16 + e >= cols) continue;
          const uint32_t key = (order16(pack_bf16x2(0.f, acc[t][mt][e]) >> 16) << 16) | (0xFFFFu - (uint32_t)local);
          best = key > best ? key : best;
        }
      auto p16 = __builtin_amdgcn_permlane16_swap(best, best, false, false);
      best = max((uint32_t)p16[0], (uint32_t)p16[1]);
      auto p32 = __builtin_amdgcn_permlane32_swap(best, best, false, false);
      best = max((uint32_t)p32[0], (uint32_t)p32[1]);
      if (g == 0) sArg[wave * TB + mt * 16 + r] = best;
    }
    __syncthreads();
    if (tid < nrows) {
      uint32_t best = sArg[tid];
#pragma unroll
      for (int w2 = 1; w2 < kLinWaves; ++w2) best = max(best, sArg[w2 * TB + tid]);
      const uint32_t col = (uint32_t)cb * kArgCols + (0xFFFFu - (best & 0xFFFFu));
      a.partial[(m0 + tid) * a.partial_stride + cb] = ((uint64_t)(best >> 16) << 32) | (uint64_t)(0xFFFFFFFFu - col);
    }
    if (advance && tid == 0) *a.pos_advance = pos_now + 1;
  }
}

// One workgroup: per row the largest of its nblk partial keys -> token; history slot *pos + 1; then *pos += 1.
// Wavefront w takes rows w, w + 16, ... four at a time, with every partial load of the four rows in flight.
constexpr int kFinishThreads = 1024;
constexpr int kFinishRows = 4;
constexpr int kFinishLoads = 4;   // partials per lane per row and round (256 blocks per round)

__global__ void __launch_bounds__(kFinishThreads)
    argmax_finish_kernel(const uint64_t *__restrict__ partial, int64_t pstride, int nblk, int64_t M,
                         int64_t *__restrict__ pos, int64_t *__restrict__ tok, int64_t *__restrict__ hist,
                         int64_t hstride, int64_t hlen, int advance) {
  constexpr int kWaves = kFinishThreads / kWave;
  const int wave = threadIdx.x / kWave, lane = lane_id();
  const int64_t P = *pos;
  for (int64_t m0 = (int64_t)wave * kFinishRows; m0 < M; m0 += (int64_t)kWaves * kFinishRows) {
    uint64_t best[kFinishRows];
#pragma unroll
    for (int i = 0; i < kFinishRows; ++i) best[i] = 0;
    for (int b0 = 0; b0 < nblk; b0 += kWave * kFinishLoads) {
      uint64_t v[kFinishRows][kFinishLoads];
#pragma unroll
      for (int i = 0; i < kFinishRows; ++i)
#pragma unroll
        for (int u = 0; u < kFinishLoads; ++u) {
          const int b = b0 + u * kWave + lane;
          const int64_t m = m0 + i < M ? m0 + i : M - 1;
          v[i][u] = partial[m * pstride + (b < nblk ? b : nblk - 1)];
        }
#pragma unroll
      for (int i = 0; i < kFinishRows; ++i)
#pragma unroll
        for (int u = 0; u < kFinishLoads; ++u) best[i] = v[i][u] > best[i] ? v[i][u] : best[i];
    }
#pragma unroll
    for (int i = 0; i < kFinishRows; ++i) {
      for (int o = kWave / 2; o > 0; o >>= 1) {
        const uint64_t other = __shfl_xor(best[i], o, kWave);
        best[i] = other > best[i] ? other : best[i];
      }
      const int64_t m = m0 + i;
      if (lane == 0 && m < M) {
        const int64_t t = (int64_t)(0xFFFFFFFFu - (uint32_t)best[i]);
        tok[m] = t;
        if (hist && P + 1 >= 0 && P + 1 < hlen) hist[m * hstride + P + 1] = t;
      }
    }
  }
  __syncthreads();  // every wavefront has read *pos
  if (advance && threadIdx.x == 0) *pos = P + 1;
}

// Launch geometry: ncb column blocks x ntg token groups of mtb tiles.
struct LinGrid {
  int ncb, ntg, mtb;
  dim3 grid;
  size_t shmem;
};

template <int PRO, int EPI, int MAXS, int MTB>
void launch_linear_mtb(const smlm_linear_args &a, const LinGrid &lg, hipStream_t stream) {
  if (PRO == SMLM_LIN_PLAIN || a.K <= 384)
    hipLaunchKernelGGL((linear_kernel<PRO, EPI, MAXS, 3, MTB>), lg.grid, dim3(kLinThreads), lg.shmem, stream, a,
                       lg.ncb, lg.ntg);
  else
    hipLaunchKernelGGL((linear_kernel<PRO, EPI, MAXS, 4, MTB>), lg.grid, dim3(kLinThreads), lg.shmem, stream, a,
                       lg.ncb, lg.ntg);
}

template <int PRO, int EPI, int MAXS>
void launch_linear_cpq(const smlm_linear_args &a, const LinGrid &lg, hipStream_t stream) {
  if constexpr (PRO == SMLM_LIN_RMSNORM_PARTS) launch_linear_mtb<PRO, EPI, MAXS, 1>(a, lg, stream);  // mtb is 1
  else if (EPI != SMLM_LIN_ARGMAX || lg.mtb == 1) launch_linear_mtb<PRO, EPI, MAXS, 1>(a, lg, stream);
  else launch_linear_mtb<PRO, EPI, MAXS, kMaxTiles>(a, lg, stream);
}

template <int PRO>
void launch_linear_pro(const smlm_linear_args &a, const LinGrid &grid, hipStream_t stream) {
  const int steps = a.K / 32;
  if constexpr (PRO != SMLM_LIN_RMSNORM_PARTS) {
    if (a.epilogue == SMLM_LIN_ARGMAX) {
      if (steps <= 12) launch_linear_cpq<PRO, SMLM_LIN_ARGMAX, 12>(a, grid, stream);
      else launch_linear_cpq<PRO, SMLM_LIN_ARGMAX, 16>(a, grid, stream);
      return;
    }
  }
  const int per_wave = (steps + kLinWaves - 1) / kLinWaves;
#define SMLM_LIN_MAXS(EPI)                                                               \
  if (per_wave == 3) launch_linear_cpq<PRO, EPI, 3>(a, grid, stream);                     \
  else if (per_wave <= 4) launch_linear_cpq<PRO, EPI, 4>(a, grid, stream);                \
  else if (PRO == SMLM_LIN_PLAIN && per_wave <= 8) launch_linear_cpq<PRO, EPI, 8>(a, grid, stream); \
  else launch_linear_cpq<PRO, EPI, 16>(a, grid, stream);
  if (a.epilogue == SMLM_LIN_STORE) {
    SMLM_LIN_MAXS(SMLM_LIN_STORE)
  } else {
    SMLM_LIN_MAXS(SMLM_LIN_SWIGLU)
  }
#undef SMLM_LIN_MAXS
}

bool aligned16(const void *p) { return ((uintptr_t)p % 16) == 0; }

}  // namespace
}  // namespace smlm

extern "C" int smlm_linear_argmax_blocks(int N) { return N <= 0 ? 0 : (N + smlm::kArgCols - 1) / smlm::kArgCols; }

extern "C" int smlm_decode_linear(const smlm_linear_args *a, void *stream) {
  using namespace smlm;
  if (!a) return fail(SMLM_EINVAL, "smlm_decode_linear: null argument block");
  const smlm_linear_args &A = *a;
  const int pro = A.prologue, epi = A.epilogue;
  if (pro != SMLM_LIN_PLAIN && pro != SMLM_LIN_RMSNORM && pro != SMLM_LIN_EMBED_RMSNORM &&
      pro != SMLM_LIN_RMSNORM_PARTS && pro != SMLM_LIN_EMBED_ARGMAX)
    return fail(SMLM_EINVAL, "smlm_decode_linear: unknown prologue %d", pro);
  if (epi != SMLM_LIN_STORE && epi != SMLM_LIN_SWIGLU && epi != SMLM_LIN_ARGMAX)
    return fail(SMLM_EINVAL, "smlm_decode_linear: unknown epilogue %d", epi);
  if (!A.w) return fail(SMLM_EINVAL, "smlm_decode_linear: null weight");
  if (A.M < 0 || A.M > (1LL << 20) || A.K < 32 || A.K % 32 || A.N < 16 || A.N % 16)
    return fail(SMLM_EINVAL, "smlm_decode_linear: bad shape M=%lld N=%d K=%d (K and N multiples of 32 and 16)",
                (long long)A.M, A.N, A.K);
  if (epi == SMLM_LIN_SWIGLU && A.N % 32)
    return fail(SMLM_EINVAL, "smlm_decode_linear: SWIGLU needs N = 2 * hidden with hidden a multiple of 16");
  const int max_k = epi == SMLM_LIN_ARGMAX ? 512 : (pro == SMLM_LIN_PLAIN ? 2048 : 512);
  if (A.K > max_k)
    return fail(SMLM_EUNSUPPORTED, "smlm_decode_linear: K=%d too large for this prologue / epilogue (at most %d)",
                A.K, max_k);
  if (!aligned16(A.w)) return fail(SMLM_EINVAL, "smlm_decode_linear: weight must be 16-byte aligned");
  if (pro == SMLM_LIN_EMBED_RMSNORM) {
    if (!A.tok || !A.emb || A.emb_rows < 1 || !aligned16(A.emb))
      return fail(SMLM_EINVAL, "smlm_decode_linear: EMBED_RMSNORM needs tok, a 16-byte aligned emb, emb_rows");
  } else if (pro == SMLM_LIN_EMBED_ARGMAX) {
    if (!A.emb || A.emb_rows < 1 || !aligned16(A.emb))
      return fail(SMLM_EINVAL, "smlm_decode_linear: EMBED_ARGMAX needs a 16-byte aligned emb and emb_rows");
    if (!A.tok_partial || !aligned16(A.tok_partial) || A.tok_blocks < 1 || A.tok_partial_stride < A.tok_blocks ||
        A.tok_partial_stride % 2)
      return fail(SMLM_EINVAL, "smlm_decode_linear: EMBED_ARGMAX needs 16-byte aligned tok_partial keys with "
                  "tok_blocks >= 1 and an even row stride >= tok_blocks");
    if (A.hist && (!A.pos || A.hist_len < 0 || A.hist_stride < A.hist_len))
      return fail(SMLM_EINVAL, "smlm_decode_linear: EMBED_ARGMAX hist needs pos and hist_stride >= hist_len >= 0");
  } else {
    if (!A.x || !aligned16(A.x) || A.x_stride < A.K || A.x_stride % 8)
      return fail(SMLM_EINVAL, "smlm_decode_linear: x must be 16-byte aligned with x_stride >= K, a multiple of 8");
  }
  if (pro != SMLM_LIN_PLAIN) {
    if (!A.norm_w || !aligned16(A.norm_w) || !(A.eps >= 0.f))
      return fail(SMLM_EINVAL, "smlm_decode_linear: the RMSNorm needs a 16-byte aligned weight and eps >= 0");
    if (A.K > 480)
      return fail(SMLM_EUNSUPPORTED, "smlm_decode_linear: normalised rows of K=%d > 480 do not fit in LDS", A.K);
    if ((A.delta && ((pro != SMLM_LIN_RMSNORM && pro != SMLM_LIN_RMSNORM_PARTS) || !aligned16(A.delta))) ||
        (A.x_out && !aligned16(A.x_out)))
      return fail(SMLM_EINVAL, "smlm_decode_linear: delta (RMSNORM prologues only) and x_out must be 16-byte aligned");
    if (pro == SMLM_LIN_RMSNORM_PARTS &&
        (!A.delta || A.delta_parts < 1 || A.delta_parts > kMaxParts || epi == SMLM_LIN_ARGMAX))
      return fail(SMLM_EINVAL, "smlm_decode_linear: RMSNORM_PARTS needs delta with 1..%d parts (delta_parts=%d) and "
                  "no ARGMAX epilogue", kMaxParts, A.delta_parts);
  } else if (A.delta || A.x_out) {
    return fail(SMLM_EINVAL, "smlm_decode_linear: delta and x_out belong to the RMSNorm prologues");
  }
  const int cols = epi == SMLM_LIN_SWIGLU ? A.N / 2 : A.N;
  if (epi == SMLM_LIN_STORE) {
    if (A.n_split < 0 || A.n_split > A.N || A.n_split % 16 || A.n_affine < 0 || A.n_affine > A.N || A.n_affine % 16)
      return fail(SMLM_EINVAL, "smlm_decode_linear: n_split and n_affine must be multiples of 16 in [0, N]");
    if ((A.n_split > 0 && (!A.out || A.out_stride < A.n_split || A.out_stride % 4 || (uintptr_t)A.out % 8)) ||
        (A.n_split < A.N && (!A.out2 || A.out2_stride < A.N - A.n_split || A.out2_stride % 4 || (uintptr_t)A.out2 % 8)))
      return fail(SMLM_EINVAL, "smlm_decode_linear: out / out2 missing, misaligned or with a short row stride");
    if (A.n_affine > 0 && (!A.scale || !A.shift))
      return fail(SMLM_EINVAL, "smlm_decode_linear: n_affine > 0 needs scale and shift");
  } else if (epi == SMLM_LIN_SWIGLU) {
    if (!A.out || A.out_stride < cols || A.out_stride % 4 || (uintptr_t)A.out % 8)
      return fail(SMLM_EINVAL, "smlm_decode_linear: SWIGLU out missing, misaligned or with a short row stride");
  } else {
    if (!A.partial || A.partial_stride < smlm_linear_argmax_blocks(A.N) || (uintptr_t)A.partial % 8)
      return fail(SMLM_EINVAL, "smlm_decode_linear: ARGMAX needs partial (M, >= %d) uint64",
                  smlm_linear_argmax_blocks(A.N));
    if (A.pos_advance && A.M == 0)
      return fail(SMLM_EINVAL, "smlm_decode_linear: pos_advance needs M >= 1 (an empty launch runs nothing)");
  }
  if (A.pos_advance && epi != SMLM_LIN_ARGMAX)
    return fail(SMLM_EINVAL, "smlm_decode_linear: pos_advance belongs to the ARGMAX epilogue");
  if (A.M == 0) return SMLM_OK;
  // 16-token groups (more workgroups, shorter per-workgroup chains: decode is latency-bound), except the ARGMAX
  // epilogue over more than 16 rows: 32-row groups (each workgroup normalises its rows in the prologue, so 64-row
  // groups measured 1% slower per batch-64 decode step; 16-row groups re-read the 24.6 MB of lm_head weights 4x),
  // and the PLAIN prologue with the STORE epilogue: 8-row groups (group_rows)
  LinGrid lg;
  lg.mtb = epi == SMLM_LIN_ARGMAX && A.M > 16 ? kMaxTiles : 1;
  const int tb = group_rows(pro, epi, lg.mtb);
  const int cols_per_block = epi == SMLM_LIN_ARGMAX ? kArgCols : 16;
  lg.ncb = (cols + cols_per_block - 1) / cols_per_block;
  lg.ntg = (int)((A.M + tb - 1) / tb);
  const int64_t nwg = lg.ntg == 1 ? lg.ncb : (int64_t)(lg.ncb + kXcds - 1) / kXcds * kXcds * lg.ntg;
  if (nwg > 0x7FFFFFFFLL)
    return fail(SMLM_EUNSUPPORTED, "smlm_decode_linear: M=%lld x N=%d needs more workgroups than one launch holds",
                (long long)A.M, A.N);
  lg.grid = dim3((unsigned)nwg);
  const int pad_rows = (int)(((A.M < tb ? A.M : tb) + 15) / 16 * 16);
  const size_t act = pro != SMLM_LIN_PLAIN ? (size_t)pad_rows * (A.K + 8) * 2 : 0;
  const size_t red = epi == SMLM_LIN_ARGMAX
                         ? (size_t)kLinWaves * tb * 4
                         : (size_t)(kLinWaves - 1) * (epi == SMLM_LIN_SWIGLU ? 2 : 1) * lg.mtb * kWave * 16;
  lg.shmem = act > red ? act : red;
  hipStream_t s = (hipStream_t)stream;
  if (pro == SMLM_LIN_PLAIN) launch_linear_pro<SMLM_LIN_PLAIN>(A, lg, s);
  else if (pro == SMLM_LIN_RMSNORM) launch_linear_pro<SMLM_LIN_RMSNORM>(A, lg, s);
  else if (pro == SMLM_LIN_RMSNORM_PARTS) launch_linear_pro<SMLM_LIN_RMSNORM_PARTS>(A, lg, s);
  else if (pro == SMLM_LIN_EMBED_RMSNORM) launch_linear_pro<SMLM_LIN_EMBED_RMSNORM>(A, lg, s);
  else launch_linear_pro<SMLM_LIN_EMBED_ARGMAX>(A, lg, s);
  return launch_status("smlm_decode_linear");
}

extern "C" int smlm_argmax_finish(const uint64_t *partial, int64_t partial_stride, int nblk, int64_t M, int64_t *pos,
                                  int64_t *tok, int64_t *hist, int64_t hist_stride, int64_t hist_len, int advance,
                                  void *stream) {
  using namespace smlm;
  if (!partial || !tok || !pos) return fail(SMLM_EINVAL, "smlm_argmax_finish: null partial, tok or pos");
  if (M < 0 || nblk < 1 || partial_stride < nblk || (hist && hist_stride < hist_len))
    return fail(SMLM_EINVAL, "smlm_argmax_finish: bad shape M=%lld nblk=%d", (long long)M, nblk);
  if (M == 0 && !advance) return SMLM_OK;
  hipLaunchKernelGGL(argmax_finish_kernel, dim3(1), dim3(kFinishThreads), 0, (hipStream_t)stream, partial,
                     partial_stride, nblk, M, pos, tok, hist, hist_stride, hist_len, advance);
  return launch_status("smlm_argmax_finish");
}
