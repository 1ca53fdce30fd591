#pragma once
// Host-callable entry points with the signatures and semantics of the
// reference's include/Kernels.hpp:9-79, so that Engine.cpp's calls compile
// against this header. Float activations are row-major device buffers;
// launches use the null stream unless a stream is given. Errors surface as the
// reference's exception types. No HIP header is included; calls go through
// the C-ABI of libqk_hip.so (include/qk_abi.h).
//
// libqk_engine.so defines every function here except rope and attention,
// which stay with the engine (they are not on the dequantize-matmul path).
#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>

#include "Weight.hpp"

namespace kernels::detail {

inline constexpr unsigned threads = 256;

// Compute units of the current device (include/Kernels.hpp:15-26).
int get_sm_count();

// Throws std::runtime_error("HIP kernel launch failed: ...") if the last
// kernel launch on this thread failed (include/Kernels.hpp:28-32), for kernels
// the engine launches itself.
void check_launch();

// Turns a C-ABI status into the reference's exceptions: invalid arguments and
// unsupported types -> std::invalid_argument (src/cuda/matmul.cu:132-136),
// launch/runtime/allocation failures -> std::runtime_error
// (include/Kernels.hpp:28-32, src/Weight.cpp:12-13).
void check_status(int status, const char* what);

}  // namespace kernels::detail

namespace kernels {

using stream_t = device_stream_t;

// Non-blocking stream (include/Kernels.hpp:38-52, src/cuda/CudaStream.cpp:13-46).
class Stream {
public:
    Stream();
    ~Stream();
    Stream(const Stream&) = delete;
    Stream& operator=(const Stream&) = delete;
    Stream(Stream&& other) noexcept;
    Stream& operator=(Stream&& other) noexcept;

    // Throws std::logic_error on a moved-from stream.
    stream_t get() const;
    void synchronize() const;
    bool ready() const;

private:
    stream_t stream_{nullptr};
};

// The reference's name for the same class.
using CudaStream = Stream;

// output = input * rsqrt(mean(input^2) + epsilon) * scale per row; scale is an
// F32 weight of `width` values (include/Kernels.hpp:54-55,
// src/cuda/rms_norm.cu:28-36). Throws std::invalid_argument for width 0, a
// non-positive epsilon or a scale that is not F32 of that width.
void rms_norm(const float* input, const Weight& scale, float* output,
    size_t rows, size_t width, float epsilon);

// output[rows x N] = Q8(input)[rows x K] . weight^T, K = weight.dimension[0],
// N = weight.dimension[1]; output is overwritten (src/cuda/matmul.cu:130-165).
void matmul(const float* input, const Weight& weight, float* output, size_t rows,
    stream_t stream = nullptr);

void matmul(const float* input, const Weight& weight, float* output, size_t rows,
    const Stream& stream);

// Rotary embedding and attention (include/Kernels.hpp:63-68): declared with
// the reference's signatures for the engine's call sites; the engine provides
// their definitions (src/cuda/rope.cu, src/cuda/attention.cu).
void rope(float* input, size_t tokens, size_t heads, size_t head_dim,
    size_t position_offset, float frequency_base);

void attention(const float* q, const float* k, const float* v, float* output,
    size_t tokens, size_t query_heads, size_t kv_heads, size_t head_dim,
    size_t query_offset = 0);

// state[i] += branch[i] (include/Kernels.hpp:70, src/cuda/residual_add.cu:15-20).
void residual_add(float* state, const float* branch, size_t count);

// out = gate/(1+exp(-gate)) * up (src/cuda/silu_multiply.cu:19-23).
void silu_multiply(const float* gate, const float* up, float* output, size_t count);

// Index of the largest logit: lowest index among equal maxima, NaN and -inf
// never win, 0xFFFFFFFF when nothing wins; blocks until the index is on the
// host (src/cuda/argmax.cu:71-98). Throws std::invalid_argument for a null
// pointer or a size outside [1, 2^32-1], std::runtime_error if the device
// collector timed out waiting for a workgroup (qk_argmax_workspace_check).
uint32_t argmax(const float* logits, size_t vocabulary_size);

// Superblock rows -> fp32 (src/cuda/embedding.cu:65-84).
void dequantize_embeddings(const void* packed, float* output, size_t rows,
    size_t width, size_t row_bytes, ggml_type type);

}  // namespace kernels
