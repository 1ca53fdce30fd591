// Exhaustive GPU check of the activation quantiser's exact-rounding helpers
// (csrc/qk_device.hpp) against IEEE float arithmetic on the same device:
//   refined_rcp(a) == 1.0f / a            for every float a in [2^-64, 2^64]
//   markstein_div(a, 127, RN(1/127)) == a / 127.0f   for the same a
//   markstein_div(x, amax, refined_rcp(amax)) == x / amax   on a sample of
//       (x, amax) pairs near code boundaries (|x| <= amax)
//   round_code(t) == (int)roundf(t)        for every float t with |t| <= 127
//   q8_code(x, amax, refined_rcp(amax)) == (int)roundf((x / amax) * 127)
//       on near-tie pairs (the composition as the kernels inline it: the
//       product fused into the rounding add would differ)
// Exits non-zero on any mismatch.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdint>

#include "qk_device.hpp"

#define CHECK(x)                                                                       \
  do {                                                                                 \
    hipError_t e_ = (x);                                                               \
    if (e_ != hipSuccess) {                                                            \
      std::printf("HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__);      \
      return 2;                                                                        \
    }                                                                                  \
  } while (0)

using qk::markstein_div;
using qk::q8_code;
using qk::refined_rcp;
using qk::round_code;

__global__ void check_divisions(uint32_t lo, uint32_t count, unsigned long long* bad) {
  unsigned long long n = 0;
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < count; i += gridDim.x * blockDim.x) {
    const float a = __builtin_bit_cast(float, lo + i);
    n += __builtin_bit_cast(uint32_t, refined_rcp(a)) != __builtin_bit_cast(uint32_t, 1.0f / a);
    n += __builtin_bit_cast(uint32_t, markstein_div(a, 127.0f, 1.0f / 127.0f)) !=
         __builtin_bit_cast(uint32_t, a / 127.0f);
  }
  if (n) atomicAdd(bad, n);
}

// (x, amax): amax from a hash-spread set, x = amax * (k + 0.5 +- tiny) / 127
// rounded, i.e. activations whose code sits next to a rounding boundary.
__global__ void check_quotients(uint32_t count, unsigned long long* bad) {
  unsigned long long n = 0;
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < count; i += gridDim.x * blockDim.x) {
    uint32_t h = i * 2654435761u;
    h ^= h >> 15;
    h *= 0x2c1b3c6du;
    h ^= h >> 12;
    const float amax = __builtin_bit_cast(float, 0x1F800000u + (h % (0x5F800000u - 0x1F800000u)));
    const int k = static_cast<int>(i % 255u) - 127;
    const float x0 = amax * ((static_cast<float>(k) + 0.5f) / 127.0f);
    for (int d = -2; d <= 2; ++d) {
      const float x = __builtin_bit_cast(float, __builtin_bit_cast(int32_t, x0) + d);
      if (!(fabsf(x) <= amax)) continue;
      const float r = refined_rcp(amax);
      n += __builtin_bit_cast(uint32_t, markstein_div(x, amax, r)) != __builtin_bit_cast(uint32_t, x / amax);
    }
  }
  if (n) atomicAdd(bad, n);
}

// The whole code formula on near-tie pairs: x = amax * (k + 0.5) / 127 and
// its neighbours, amax from a hash-spread set or a small integer, plus small
// integer activations against an integer maximum (x = 1, amax = 254: RN(1/254)
// * 127 rounds up to exactly 0.5, code 1).
__global__ void check_codes(uint32_t count, unsigned long long* bad) {
  unsigned long long n = 0;
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < count; i += gridDim.x * blockDim.x) {
    uint32_t h = i * 2246822519u;
    h ^= h >> 13;
    h *= 0x5bd1e995u;
    h ^= h >> 15;
    const float amax = (i & 1u) ? static_cast<float>(1u + (h % 4096u))
                                : __builtin_bit_cast(float, 0x1F800000u + (h % (0x5F800000u - 0x1F800000u)));
    const int k = static_cast<int>((i >> 1) % 255u) - 127;
    const float x0 = amax * ((static_cast<float>(k) + 0.5f) / 127.0f);
    const float r = refined_rcp(amax);
    for (int d = -2; d <= 2; ++d) {
      const float x = __builtin_bit_cast(float, __builtin_bit_cast(int32_t, x0) + d);
      if (!(fabsf(x) <= amax)) continue;
      n += q8_code(x, amax, r) != static_cast<int>(roundf((x / amax) * 127.0f));
    }
    if (i & 1u) {
      const float xi = static_cast<float>(static_cast<int>(h >> 20) % (static_cast<int>(amax) + 1));
      n += q8_code(xi, amax, r) != static_cast<int>(roundf((xi / amax) * 127.0f));
    }
  }
  if (n) atomicAdd(bad, n);
}

__global__ void check_rounding(uint32_t count, unsigned long long* bad) {
  unsigned long long n = 0;
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < count; i += gridDim.x * blockDim.x) {
    // every non-negative float <= 127 and its negation
    const float t = __builtin_bit_cast(float, i);
    n += round_code(t) != static_cast<int>(roundf(t));
    n += round_code(-t) != static_cast<int>(roundf(-t));
  }
  if (n) atomicAdd(bad, n);
}

int main() {
  unsigned long long* bad = nullptr;
  CHECK(hipMalloc(&bad, 4 * sizeof(unsigned long long)));
  CHECK(hipMemset(bad, 0, 4 * sizeof(unsigned long long)));
  const uint32_t lo = 0x1F800000u, hi = 0x5F800000u;  // 2^-64 .. 2^64
  const uint32_t t127 = 0x42FE0000u;                  // 127.0f
  check_divisions<<<4096, 256>>>(lo, hi - lo + 1, bad);
  check_quotients<<<4096, 256>>>(1u << 26, bad + 1);
  check_rounding<<<4096, 256>>>(t127 + 1, bad + 2);
  check_codes<<<4096, 256>>>(1u << 26, bad + 3);
  CHECK(hipGetLastError());
  CHECK(hipDeviceSynchronize());
  unsigned long long h[4];
  CHECK(hipMemcpy(h, bad, sizeof(h), hipMemcpyDeviceToHost));
  std::printf("reciprocal and a/127 over [2^-64, 2^64]: %llu mismatches\n", h[0]);
  std::printf("x/amax near code boundaries (2^26 pairs x 5): %llu mismatches\n", h[1]);
  std::printf("roundf over |t| <= 127: %llu mismatches\n", h[2]);
  std::printf("codes roundf(x/amax*127) near ties (2^26 pairs): %llu mismatches\n", h[3]);
  CHECK(hipFree(bad));
  return h[0] || h[1] || h[2] || h[3] ? 1 : 0;
}
