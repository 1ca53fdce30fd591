// Q8 activation quantisation: fp32 [M x K] -> qk_q8_block per 32 activations.
// Arithmetic of src/cuda/matmul.cu:8-22 (amax over 32, scale = amax/127,
// code = roundf((x/amax)*127)), plus the per-block code sums that the
// superblock dots consume (Q4_K min term, Q6_K -32 offset).
#include "qk_device.hpp"
#include "qk_launch.hpp"

namespace qk {
namespace {

// One activation per lane; a 32-lane half-wave owns one Q8 block, so the
// reductions stay inside the half-wave (xor offsets < 32).
__global__ __launch_bounds__(256) void quantize_q8_kernel(const float* __restrict__ x,
                                                          qk_q8_block* __restrict__ out,
                                                          int64_t count) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= count) return;  // count % 32 == 0: half-waves exit whole
  const float v = x[i];
  float amax = fabsf(v);
#pragma unroll
  for (int o = 16; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 32));
  const float scale = amax / 127.0f;
  const int code = amax == 0.0f ? 0 : static_cast<int>(roundf((v / amax) * 127.0f));
  int s16 = code;
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) s16 += __shfl_xor(s16, o, 32);
  const int s_other = __shfl_xor(s16, 16, 32);
  const int lane = threadIdx.x & 31;
  qk_q8_block* blk = out + (i >> 5);
  blk->codes[lane] = static_cast<int8_t>(code);
  if (lane == 0) {
    blk->scale = scale;
    blk->scaled_sum = scale * static_cast<float>(s16 + s_other);
    blk->neg32_sum_lo = -32 * s16;
    blk->neg32_sum_hi = -32 * s_other;
  }
}

}  // namespace

hipError_t launch_quantize_q8(const float* x, int64_t M, int64_t K, qk_q8_block* q8,
                              hipStream_t stream) {
  const int64_t count = M * K;
  const int64_t blocks = (count + 255) / 256;
  quantize_q8_kernel<<<dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, stream>>>(x, q8,
                                                                                   count);
  return hipGetLastError();
}

}  // namespace qk
