// out = gate/(1+exp(-gate)) * up (src/cuda/silu_multiply.cu:6-12), with the
// ROCm device library's expf; the row-wise RMSNorm (src/cuda/rms_norm.cu:6-24)
// with its rsqrtf; and state += branch (src/cuda/residual_add.cu:6-9).
#include "qk_device.hpp"
#include "qk_launch.hpp"

namespace qk {
namespace {

__global__ __launch_bounds__(256) void silu_multiply_kernel(const float* __restrict__ gate,
                                                            const float* __restrict__ up,
                                                            float* __restrict__ out,
                                                            int64_t count) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < count; i += stride) {
    const float g = gate[i];
    out[i] = (g / (1.0f + expf(-g))) * up[i];
  }
}

// out = x * rsqrt(mean(x^2) + eps) * scale for one row per workgroup (the
// mat-vec's RMSNorm fold does the same inside its prologue at M = 1).
__global__ __launch_bounds__(256) void rms_norm_kernel(const float* __restrict__ x,
                                                       const float* __restrict__ scale,
                                                       float* __restrict__ out, int width,
                                                       float eps) {
  __shared__ float partial[4];
  const float* xr = x + static_cast<int64_t>(blockIdx.x) * width;
  float* o = out + static_cast<int64_t>(blockIdx.x) * width;
  const int tid = static_cast<int>(threadIdx.x);
  float sum = 0.0f;
  for (int i = tid; i < width; i += 256) sum += xr[i] * xr[i];
  for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
  if ((tid & 63) == 0) partial[tid >> 6] = sum;
  __syncthreads();
  const float total = (partial[0] + partial[1]) + (partial[2] + partial[3]);
  const float inv = rsqrtf(total / static_cast<float>(width) + eps);
  for (int i = tid; i < width; i += 256) o[i] = (xr[i] * inv) * scale[i];
}

__global__ __launch_bounds__(256) void residual_add_kernel(float* __restrict__ state,
                                                           const float* __restrict__ branch,
                                                           int64_t count) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < count; i += stride)
    state[i] += branch[i];
}

}  // namespace

hipError_t launch_residual_add(float* state, const float* branch, int64_t count,
                               hipStream_t stream) {
  const int64_t blocks = (count + 255) / 256;
  const uint32_t grid = static_cast<uint32_t>(blocks < 16384 ? blocks : 16384);
  residual_add_kernel<<<grid, 256, 0, stream>>>(state, branch, count);
  return hipGetLastError();
}

hipError_t launch_rms_norm(const float* x, const float* scale, float* out, int64_t rows,
                           int64_t width, float eps, hipStream_t stream) {
  rms_norm_kernel<<<static_cast<uint32_t>(rows), 256, 0, stream>>>(x, scale, out,
                                                                   static_cast<int>(width), eps);
  return hipGetLastError();
}

hipError_t launch_silu_multiply(const float* gate, const float* up, float* out, int64_t count,
                                hipStream_t stream) {
  const int64_t blocks = (count + 255) / 256;
  const uint32_t grid = static_cast<uint32_t>(blocks < 16384 ? blocks : 16384);
  silu_multiply_kernel<<<grid, 256, 0, stream>>>(gate, up, out, count);
  return hipGetLastError();
}

}  // namespace qk
