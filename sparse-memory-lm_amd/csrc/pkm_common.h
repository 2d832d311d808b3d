// Shared helpers of the gfx950 product-key-memory kernels: bit-exact bf16 rounding, order-preserving score
// codes, wavefront primitives and the error state of the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "smlm_pkm.h"

namespace smlm {

constexpr int kWave = 64;  // CDNA wavefront width

// ---- error state (one message per host thread) -------------------------------------------------------------
int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
int launch_status(const char *what);  // hipGetLastError() after a launch -> SMLM_OK / SMLM_EHIP
void clear_error();

inline bool is_pow2(int64_t x) { return x > 0 && (x & (x - 1)) == 0; }

// ---- number formats ------------------------------------------------------------------------------------------
// fp32 -> bf16 bit pattern, round to nearest even, done on the integer bits so that every device and the CPU
// oracle round identically (the convention of smlm/kernels.py:106-112).
__device__ __forceinline__ uint32_t bf16_bits_rtne(float x) {
  uint32_t u = __float_as_uint(x);
  u = u + 0x7FFFu + ((u >> 16) & 1u);
  return u >> 16;
}
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) { return __uint_as_float(b << 16); }
__device__ __forceinline__ float round_bf16(float x) { return bf16_bits_to_f32(bf16_bits_rtne(x)); }

// Two fp32 values as packed bf16 bits (a in bits 0-15), round to nearest even, in one v_cvt_pk_bf16_f32: the same
// bits as bf16_bits_rtne for every finite value and infinity (a NaN becomes a quiet NaN).  For arithmetic whose
// values are finite (the LM's activations); the selection keeps the integer definition above.
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
}
__device__ __forceinline__ float round_bf16_hw(float x) { return __uint_as_float(pack_bf16x2(0.f, x) & 0xFFFF0000u); }

__device__ __forceinline__ float f16_bits_to_f32(uint16_t b) { return (float)__builtin_bit_cast(_Float16, b); }
// fp32 -> fp16 bit pattern, round to nearest even (v_cvt_f16_f32)
__device__ __forceinline__ uint16_t f32_to_f16_bits(float x) { return __builtin_bit_cast(uint16_t, (_Float16)x); }

// Order-preserving unsigned codes: a > b as floats  <=>  code(a) > code(b) as unsigned integers, with -0 ranked
// just below +0 (the convention of smlm/kernels.py:114-126).
__device__ __forceinline__ uint32_t order16(uint32_t b) { return (b & 0x8000u) ? (~b & 0xFFFFu) : (b | 0x8000u); }
__device__ __forceinline__ uint32_t unorder16(uint32_t o) { return (o & 0x8000u) ? (o ^ 0x8000u) : (~o & 0xFFFFu); }
__device__ __forceinline__ uint32_t order32(uint32_t u) { return (u & 0x80000000u) ? ~u : (u | 0x80000000u); }
__device__ __forceinline__ uint32_t unorder32(uint32_t o) { return (o & 0x80000000u) ? (o ^ 0x80000000u) : ~o; }

// ---- wavefront primitives --------------------------------------------------------------------------------
__device__ __forceinline__ int lane_id() { return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0)); }
__device__ __forceinline__ uint64_t ballot(bool p) { return __ballot(p); }
// number of set bits of `mask` below this lane
__device__ __forceinline__ int lanes_below(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0));
}
// Orders this wave's LDS accesses for the compiler; the LDS itself executes one wave's instructions in order.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ float wave_sum(float v) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

// v of lane ^ J (J < 64) on every lane: quad permutes (1, 2), two row rotations that each write half of the lanes
// (4), a row rotation (8), and the gfx950 permlane swaps (16, 32), which given a register twice return v[lane] and
// v[lane ^ J] in some order.  The DPP moves have every lane either read a valid source lane or be rewritten by the
// second move, so they need no initial value in the destination (one instruction each, no zero fill).
template <int J>
__device__ __forceinline__ uint32_t xor_lane(uint32_t v) {
  const int lane = lane_id();
  if constexpr (J == 1) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, false);  // quad_perm [1, 0, 3, 2]
  } else if constexpr (J == 2) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, false);  // quad_perm [2, 3, 0, 1]
  } else if constexpr (J == 4) {
    // row_ror:n has lane i of a row read lane (i - n) mod 16: n = 12 is i + 4 for banks 0 and 2 (lanes 0-3,
    // 8-11 of the row), n = 4 is i - 4 for banks 1 and 3; the bank mask keeps each move to its lanes
    const int t = __builtin_amdgcn_mov_dpp((int)v, 0x12C, 0xF, 0x5, false);
    return (uint32_t)__builtin_amdgcn_update_dpp(t, (int)v, 0x124, 0xF, 0xA, false);
  } else if constexpr (J == 8) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x128, 0xF, 0xF, false);  // row_ror:8
  } else if constexpr (J == 16) {
    const auto p = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return (lane & 16) ? (uint32_t)p[0] : (uint32_t)p[1];
  } else {
    const auto p = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return (lane & 32) ? (uint32_t)p[0] : (uint32_t)p[1];
  }
}

template <int J>
__device__ __forceinline__ uint64_t xor_lane64(uint64_t v) {
  return (uint64_t)xor_lane<J>((uint32_t)v) | ((uint64_t)xor_lane<J>((uint32_t)(v >> 32)) << 32);
}

}  // namespace smlm
