// Device-wide argmax with the reference's candidate rules
// (src/cuda/argmax.cu:13-23,32): the largest score wins, ties go to the
// lowest index, NaN and -inf never win (the candidate starts at -inf and is
// replaced only by a strictly greater score), and when nothing wins the
// result is SIZE_MAX truncated to uint32_t, 0xFFFFFFFF (:96).
//
// Candidates are 64-bit keys whose unsigned order is that rule: high word =
// the score's bits mapped to an order-preserving unsigned value (-0 folded
// onto +0, which compare equal), low word = ~index; key 0 = "no candidate".
// Every workgroup reduces its keys and publishes one partial; the first
// workgroup collects them and writes the index.
#pragma once

#include "qk_device.hpp"

namespace qk {

constexpr int kArgmaxSlots = 1024;  // workgroups one launch may use
// Bound of the collector's wait for one partial: 0.2 s of the 100 MHz
// real-time clock (every workgroup runs to completion without waiting, so
// only a device too busy to start a workgroup for that long reaches it).
constexpr uint64_t kArgmaxSpinTicks = 20000000;

// Caller-owned, zero-filled once before its first use; every launch leaves
// the slots at zero again. One workspace per concurrently running launch.
struct ArgmaxWorkspace {
  uint64_t partial[kArgmaxSlots];  // workgroup b's best key + 1; 0 = not yet published
  uint32_t timeout;                // set if the collector stopped waiting (that index is invalid)
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
// flow, with the thread's best key. `lds` holds at least `waves` keys. Every
// workgroup but the first publishes its best key + 1 (keys stay below 2^64-1)
// with one agent-scope coherent store and exits; workgroup 0, after its own
// share, polls the slots with agent-scope coherent loads until each is
// non-zero, reduces them with its own keys, writes the index and clears the
// slots for the next launch. No atomics and no cache maintenance: the chain
// after the last workgroup's rows is one store reaching memory and one poll
// (an arrival counter cost two more round trips, release/acquire fences at
// agent scope an L2 write-back and invalidate each on MI355X). The collector
// only waits for stores that are already issued or for workgroups that run
// without waiting, so its bounded wait ends in practice long before its limit.
__device__ __forceinline__ void argmax_finish(uint64_t key, ArgmaxWorkspace* __restrict__ ws,
                                              uint32_t* __restrict__ result, uint64_t* lds,
                                              int waves) {
  key = wave_max_key(key);
  const int wave = static_cast<int>(threadIdx.x >> 6);
  if ((threadIdx.x & 63u) == 0) lds[wave] = key;
  __syncthreads();
  uint64_t best = 0;
  if (threadIdx.x == 0)
    for (int i = 0; i < waves; ++i) best = max_key(best, lds[i]);
  if (blockIdx.x != 0) {
    if (threadIdx.x == 0)
      __hip_atomic_store(&ws->partial[blockIdx.x], best + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  for (uint32_t i = 1 + threadIdx.x; i < gridDim.x; i += blockDim.x) {
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    uint64_t v;
    while ((v = __hip_atomic_load(&ws->partial[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) == 0) {
      if (__builtin_amdgcn_s_memrealtime() - t0 > kArgmaxSpinTicks) {
        __hip_atomic_store(&ws->timeout, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    if (v != 0) best = max_key(best, v - 1);
    __hip_atomic_store(&ws->partial[i], uint64_t{0}, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  best = wave_max_key(best);
  __syncthreads();  // thread 0 has read the keys of the first round
  if ((threadIdx.x & 63u) == 0) lds[wave] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int i = 0; i < waves; ++i) best = max_key(best, lds[i]);
    *result = argmax_index(best);
  }
}

}  // namespace qk
