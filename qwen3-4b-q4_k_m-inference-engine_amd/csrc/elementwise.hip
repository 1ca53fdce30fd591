// out = gate/(1+exp(-gate)) * up (src/cuda/silu_multiply.cu:6-12), with the
// ROCm device library's expf.
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

}  // namespace

hipError_t launch_silu_multiply(const float* gate, const float* up, float* out, int64_t count,
                                hipStream_t stream) {
  const int64_t blocks = (count + 255) / 256;
  const uint32_t grid = static_cast<uint32_t>(blocks < 16384 ? blocks : 16384);
  silu_multiply_kernel<<<grid, 256, 0, stream>>>(gate, up, out, count);
  return hipGetLastError();
}

}  // namespace qk
