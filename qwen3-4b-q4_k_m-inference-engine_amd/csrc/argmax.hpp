// Device-wide argmax with the reference's candidate rules
// (src/cuda/argmax.cu:13-23,32): the largest score wins, ties go to the
// lowest index, NaN and -inf never win (the candidate starts at -inf and is
// replaced only by a strictly greater score), and when nothing wins the
// result is SIZE_MAX truncated to uint32_t, 0xFFFFFFFF (:96).
//
// Candidates are 64-bit keys whose unsigned order is that rule: high word =
// the score's bits mapped to an order-preserving unsigned value (-0 folded
// onto +0, which compare equal), low word = ~index; key 0 = "no candidate".
// Every workgroup reduces its keys, publishes one partial with a release,
// and the last workgroup to arrive (agent-scope arrival counter) reduces the
// partials, writes the index and re-arms the counter for the next launch.
#pragma once

#include "qk_device.hpp"

namespace qk {

constexpr int kArgmaxSlots = 1024;  // workgroups one launch may use

// Caller-owned, zero-filled once before its first use; every launch leaves
// the counter at zero again. One workspace per concurrently running launch.
struct ArgmaxWorkspace {
  uint64_t partial[kArgmaxSlots];
  uint32_t arrivals;
  uint32_t pad[3];
};

__device__ __forceinline__ uint64_t argmax_key(float v, uint32_t index) {
  if (!(v > -__builtin_inff())) return 0;                        // NaN, -inf
  const uint32_t b = __builtin_bit_cast(uint32_t, v + 0.0f);     // -0 -> +0
  const uint32_t ord = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return (static_cast<uint64_t>(ord) << 32) | (0xFFFFFFFFu - index);
}

__device__ __forceinline__ uint32_t argmax_index(uint64_t key) {
  return key ? 0xFFFFFFFFu - static_cast<uint32_t>(key) : 0xFFFFFFFFu;
}

__device__ __forceinline__ uint64_t max_key(uint64_t a, uint64_t b) { return a > b ? a : b; }

__device__ __forceinline__ uint64_t wave_max_key(uint64_t k) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) k = max_key(k, __shfl_xor(k, off));
  return k;
}

// Called by every thread of every workgroup of the launch, in uniform control
// flow, with the thread's best key. `lds` holds at least waves + 1 keys.
__device__ __forceinline__ void argmax_finish(uint64_t key, ArgmaxWorkspace* __restrict__ ws,
                                              uint32_t* __restrict__ result, uint64_t* lds,
                                              int waves) {
  key = wave_max_key(key);
  const int wave = static_cast<int>(threadIdx.x >> 6);
  if ((threadIdx.x & 63u) == 0) lds[wave] = key;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t best = 0;
    for (int i = 0; i < waves; ++i) best = max_key(best, lds[i]);
    ws->partial[blockIdx.x] = best;
    // release: the partial is visible before the arrival is counted
    const uint32_t ticket =
        __hip_atomic_fetch_add(&ws->arrivals, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    lds[waves] = ticket == gridDim.x - 1 ? 1u : 0u;
  }
  __syncthreads();
  if (lds[waves] == 0) return;  // workgroup-uniform
  // the last workgroup: every other partial has been released
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  uint64_t best = 0;
  for (uint32_t i = threadIdx.x; i < gridDim.x; i += blockDim.x)
    best = max_key(best, __hip_atomic_load(&ws->partial[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
  best = wave_max_key(best);
  __syncthreads();  // everyone has read lds[waves]
  if ((threadIdx.x & 63u) == 0) lds[wave] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int i = 0; i < waves; ++i) best = max_key(best, lds[i]);
    *result = argmax_index(best);
    __hip_atomic_store(&ws->arrivals, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

}  // namespace qk
