// Q8 activation quantisation: fp32 [M x K] -> qk_q8_block per 32 activations.
// Arithmetic of src/cuda/matmul.cu:8-22 (amax over 32, scale = amax/127,
// code = roundf((x/amax)*127)), plus the per-block code sums that the
// superblock dots consume (Q4_K min term, Q6_K -32 offset).
#include "gemv_kernel.hpp"
#include "qk_launch.hpp"

namespace qk {
namespace {

// Eight activations per lane (two 16-byte loads); the four lanes of a quad
// own one Q8 block and reduce with DPP inside the quad, through the
// mat-vec prologue's quantiser (quantize_quarter: the reference's IEEE
// quotients and roundf, exactly). Lane 0 of the quad writes the block's
// 16-byte record. At 8 x 9728 activations (the batched FFN's h: 38
// workgroups) a kernel trace puts it at 5.1 us, the same as one activation
// per lane with shuffle reductions: the launch is latency-bound (a 3-workgroup
// buffer fill takes 3.0 us in the same trace), not VALU-bound.
__global__ __launch_bounds__(256) void quantize_q8_kernel(const float* __restrict__ x,
                                                          qk_q8_block* __restrict__ out,
                                                          int64_t tasks) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (t >= tasks) return;  // tasks % 4 == 0: quads exit whole
  const f32x4 a = *reinterpret_cast<const f32x4_a4*>(x + 8 * t);
  const f32x4 b = *reinterpret_cast<const f32x4_a4*>(x + 8 * t + 4);
  const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  store_q8_quarter(out + (t >> 2), static_cast<uint32_t>(t & 3), quantize_quarter(v));
}

}  // namespace

hipError_t launch_quantize_q8(const float* x, int64_t M, int64_t K, qk_q8_block* q8,
                              hipStream_t stream) {
  const int64_t tasks = M * K / 8;
  const int64_t blocks = (tasks + 255) / 256;
  quantize_q8_kernel<<<dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, stream>>>(x, q8, tasks);
  return hipGetLastError();
}

}  // namespace qk
