// Standalone device argmax over fp32 logits (replaces kernels::argmax,
// include/Kernels.hpp:77, src/cuda/argmax.cu:71-98, without its blocking copy
// of per-SM candidates: the last workgroup writes the index to device memory).
#include <cstddef>

#include "argmax.hpp"
#include "qk_launch.hpp"

namespace qk {
namespace {

constexpr int kArgmaxWaves = 16;

__global__ __launch_bounds__(64 * kArgmaxWaves) void argmax_kernel(const float* __restrict__ v,
                                                                   int64_t count,
                                                                   ArgmaxWorkspace* ws,
                                                                   uint32_t* result) {
  __shared__ uint64_t keys[kArgmaxWaves + 1];
  uint64_t best = 0;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 64 * kArgmaxWaves;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 64 * kArgmaxWaves + threadIdx.x; i < count;
       i += stride)
    best = max_key(best, argmax_key(v[i], static_cast<uint32_t>(i)));
  argmax_finish(best, ws, result, keys, kArgmaxWaves);
}

}  // namespace

size_t argmax_workspace_bytes() { return sizeof(ArgmaxWorkspace); }
size_t argmax_timeout_offset() { return offsetof(ArgmaxWorkspace, timeout); }
size_t argmax_slots_bytes() { return sizeof(ArgmaxWorkspace::partial); }

hipError_t launch_argmax(const float* logits, int64_t count, void* workspace, uint32_t* result,
                         hipStream_t stream) {
  int device = 0, cus = 0;
  hipError_t e = hipGetDevice(&device);
  if (e != hipSuccess) return e;
  e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device);
  if (e != hipSuccess) return e;
  const int64_t per_block = 64 * kArgmaxWaves;
  int64_t grid = (count + per_block - 1) / per_block;
  grid = grid < cus ? grid : cus;
  grid = grid < kArgmaxSlots ? grid : kArgmaxSlots;
  argmax_kernel<<<static_cast<uint32_t>(grid), 64 * kArgmaxWaves, 0, stream>>>(
      logits, count, static_cast<ArgmaxWorkspace*>(workspace), result);
  return hipGetLastError();
}

}  // namespace qk
