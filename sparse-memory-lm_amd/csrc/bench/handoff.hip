// Measurement kernels for bench.py (built into libsmlm_bench.so, not part of the lookup library): the cost of a
// dependent stage when workgroups hand data to each other, by a kernel boundary or by a device-side handoff
// inside one persistent kernel.
//
// A stage: every workgroup (64 threads) reads the whole vector of kVec floats that the previous stage wrote,
// sums it, and writes its own kVec / nwg elements of the next vector (double-buffered).  That is the shape of a
// decode step's dependent kernels (each needs all of its predecessor's output).  Variants:
//   chain       one kernel per stage; the caller captures `stages` launches in a HIP graph;
//   persistent  one kernel runs all stages, with a handoff between them:
//     kind 0  one counter, each workgroup adds 1 (release) and waits for epoch * nwg;
//     kind 1  8 group counters (workgroup % 8, the dispatcher's XCD order), whose last arrival adds 1 to a
//             top counter (release); all wait for epoch * 8 on the top counter;
//     kind 2  a flag per workgroup, stored with release, all polled by every workgroup;
//     kind 3  as 2, but the data is written and read with device-coherent accesses, so no cache writeback or
//             invalidate is needed: the flag is stored after the wavefront's data stores have completed.
//   Kinds 0-2 end a wait with an acquire fence.
// Every wait is bounded: after kSpin polls, or once any workgroup has given up, a workgroup sets the abort flag
// and returns, so the kernel always drains.  The host reads the abort flag after the run and can also set it
// before a launch to stop every wait at its first poll.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

constexpr int kVec = 512;
constexpr uint32_t kSpin = 1u << 20;

__device__ __forceinline__ void stage(const float *vin, float *vout, int wg, int nwg, int st) {
  float s = 0.f;
  for (int i = threadIdx.x; i < kVec; i += 64) s += __hip_atomic_load(vin + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
  const int per = kVec / nwg;
  if (threadIdx.x < per)
    __hip_atomic_store(vout + wg * per + threadIdx.x, s * 1e-3f + (float)st, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

__global__ void __launch_bounds__(64) chain_kernel(const float *vin, float *vout, int st) {
  stage(vin, vout, blockIdx.x, gridDim.x, st);
}

__device__ __forceinline__ bool should_stop(uint32_t n, const uint32_t *abort) {
  return n > kSpin || __hip_atomic_load(abort, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
}

// false: this workgroup gave up (its wait ran out, or another workgroup's did)
__device__ bool handoff(int kind, uint32_t *ctr, uint32_t *flags, uint32_t *abort, int wg, int nwg, uint32_t epoch) {
  bool ok = true;
  if (kind <= 1) {
    if (threadIdx.x == 0) {
      uint32_t target;
      if (kind == 0) {
        __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
        target = epoch * (uint32_t)nwg;
      } else {
        const uint32_t per_group = (uint32_t)nwg / 8;
        uint32_t *group = ctr + 64 * (1 + (wg & 7));  // one 256-byte line per counter
        const uint32_t old = __hip_atomic_fetch_add(group, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        if (old == epoch * per_group - 1) __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
        target = epoch * 8u;
      }
      uint32_t n = 0;
      while (__hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
        if (should_stop(++n, abort)) {
          ok = false;
          break;
        }
      }
      if (!ok) __hip_atomic_store(abort, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  } else {
    if (kind == 3) {
      __builtin_amdgcn_s_waitcnt(0);  // this wavefront's data stores have completed
      if (threadIdx.x == 0) __hip_atomic_store(flags + wg, epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else if (threadIdx.x == 0) {
      __hip_atomic_store(flags + wg, epoch, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
    }
    uint32_t n = 0;
    for (;;) {
      bool seen = true;
      for (int i = threadIdx.x; i < nwg; i += 64)
        seen = seen && __hip_atomic_load(flags + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= epoch;
      if (__builtin_amdgcn_ballot_w64(!seen) == 0) break;
      if (__builtin_amdgcn_readfirstlane((int)should_stop(++n, abort))) {
        ok = false;
        break;
      }
    }
    if (!ok && threadIdx.x == 0) __hip_atomic_store(abort, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (kind != 3) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  return __builtin_amdgcn_readfirstlane((int)ok) != 0;  // the workgroup is one wavefront
}

__global__ void __launch_bounds__(64) persistent_kernel(float *v0, float *v1, int stages, int kind, uint32_t *ctr,
                                                        uint32_t *flags, uint32_t *abort) {
  const int wg = blockIdx.x, nwg = gridDim.x;
  for (int st = 0; st < stages; ++st) {
    stage((st & 1) ? v1 : v0, (st & 1) ? v0 : v1, wg, nwg, st);
    if (!handoff(kind, ctr, flags, abort, wg, nwg, (uint32_t)st + 1)) return;
  }
}

bool valid_grid(int nwg) { return nwg >= 8 && nwg <= 256 && nwg % 8 == 0 && kVec % nwg == 0; }

}  // namespace

extern "C" {

// Vector length of a stage (floats): v0 and v1 hold this many.
int smlm_bench_handoff_vec(void) { return kVec; }

// `stages` dependent stage kernels of nwg workgroups, alternating v0 -> v1 -> v0 ...
int smlm_bench_handoff_chain(float *v0, float *v1, int stages, int nwg, void *stream) {
  if (!v0 || !v1 || stages < 1 || !valid_grid(nwg)) return -1;
  for (int st = 0; st < stages; ++st)
    hipLaunchKernelGGL(chain_kernel, dim3(nwg), dim3(64), 0, (hipStream_t)stream, (st & 1) ? v1 : v0,
                       (st & 1) ? v0 : v1, st);
  return hipGetLastError() == hipSuccess ? 0 : -3;
}

// The same stages in one persistent kernel with handoff `kind` (0-3).  ctr: 576 zeroed uint32; flags: nwg zeroed
// uint32; abort: one uint32, 0 to run (read it afterwards: 1 = a wait gave up and the results are incomplete).
// All nwg <= 256 single-wavefront workgroups fit the chip at once, so every wait is met unless aborted.
int smlm_bench_handoff_persistent(float *v0, float *v1, int stages, int nwg, int kind, uint32_t *ctr,
                                  uint32_t *flags, uint32_t *abort, void *stream) {
  if (!v0 || !v1 || !ctr || !flags || !abort || stages < 1 || kind < 0 || kind > 3 || !valid_grid(nwg)) return -1;
  hipLaunchKernelGGL(persistent_kernel, dim3(nwg), dim3(64), 0, (hipStream_t)stream, v0, v1, stages, kind, ctr,
                     flags, abort);
  return hipGetLastError() == hipSuccess ? 0 : -3;
}

}  // extern "C"
