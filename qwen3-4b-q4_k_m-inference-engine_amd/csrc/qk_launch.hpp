// Internal launchers shared by the kernel translation units and the C-ABI
// layer. Every launcher enqueues on `stream` and returns the hipError_t of
// the launch; shapes are validated by the caller (abi.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "qk_abi.h"

namespace qk {

hipError_t launch_quantize_q8(const float* x, int64_t M, int64_t K, qk_q8_block* q8,
                              hipStream_t stream);

hipError_t launch_gemv(const qk_q8_block* q8, const void* w, int type, int64_t K, int64_t N,
                       float* y, int64_t M, hipStream_t stream);

hipError_t launch_dequantize_rows(const void* packed, float* out, int64_t rows, int64_t K,
                                  size_t row_bytes, int type, hipStream_t stream);

hipError_t launch_silu_multiply(const float* gate, const float* up, float* out, int64_t count,
                                hipStream_t stream);

hipError_t launch_synth_superblocks(void* w, int type, int64_t N, int64_t K, uint64_t seed,
                                    float dmax, float dminmax, hipStream_t stream);

hipError_t launch_synth_normal(float* x, int64_t count, uint64_t seed, hipStream_t stream);

}  // namespace qk
