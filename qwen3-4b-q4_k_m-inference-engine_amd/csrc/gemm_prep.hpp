// Activation prep arithmetic of the prefill GEMM, shared by the prep kernel
// (gemm.hip) and the short-prompt GEMM that forms its own planes
// (gemm_kquant.hip): the Q8 round trip of x (MatmulReference.hpp:11-29:
// round(x/amax*127) * (amax/127) per 32 values), scaled by a power of two,
// split into two fp16 planes hi + lo with hi = fp16(v), lo = fp16(v - hi).
#pragma once

#include "qk_device.hpp"

namespace qk {

typedef _Float16 half2v __attribute__((ext_vector_type(2)));

constexpr int kHeadroomExp = 14;          // scaled magnitudes below 2^15 < fp16 max

// Power-of-two exponent that brings a positive finite bound into
// [2^14, 2^15); 0 for 0, clamped for inf/nan bounds (their products are
// inf/nan whatever the scale).
__device__ __forceinline__ int headroom_exponent(float bound) {
  if (!(bound > 0.0f)) return 0;
  if (!(bound <= 3.0e38f)) return -64;
  return min(kHeadroomExp - ilogbf(bound), 100);  // 2^s and 2^-s stay normal floats
}

__device__ __forceinline__ uint32_t pack2(float a, float b) {
  return __builtin_bit_cast(uint32_t, half2v{static_cast<_Float16>(a), static_cast<_Float16>(b)});
}

// v -> (fp16(v), fp16(v - fp16(v))) for a pair of values, packed.
__device__ __forceinline__ void split2(float a, float b, uint32_t& hi, uint32_t& lo) {
  const _Float16 ha = static_cast<_Float16>(a), hb = static_cast<_Float16>(b);
  hi = __builtin_bit_cast(uint32_t, half2v{ha, hb});
  lo = pack2(a - static_cast<float>(ha), b - static_cast<float>(hb));
}

// One lane's 8 values of a 32-value block with maximum |x| = bmax: the codes
// and scale as the reference computes them in float (for bmax in [2^-64,
// 2^64] through the exact reciprocal and Markstein quotient of the mat-vec
// quantiser, equal to IEEE division), v = (code * scale) * up split into fp16
// pairs h / l, and the sum of the 8 v in order.
__device__ __forceinline__ void q8_scaled_planes(const float (&v)[8], float bmax, float up, uint32_t (&h)[4],
                                                 uint32_t (&l)[4], float& sum) {
  float code[8], scale;
  if (bmax >= 0x1p-64f && bmax <= 0x1p64f) {
    const float r = refined_rcp(bmax);
#pragma unroll
    for (int i = 0; i < 8; ++i) code[i] = static_cast<float>(q8_code(v[i], bmax, r));
    scale = markstein_div(bmax, 127.0f, 1.0f / 127.0f);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) code[i] = bmax == 0.0f ? 0.0f : roundf((v[i] / bmax) * 127.0f);
    scale = bmax / 127.0f;
  }
  sum = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float c0 = code[2 * i], c1 = code[2 * i + 1];
    const float s0 = (c0 * scale) * up, s1 = (c1 * scale) * up;
    split2(s0, s1, h[i], l[i]);
    sum += s0;
    sum += s1;
  }
}

}  // namespace qk
