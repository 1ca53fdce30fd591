// kernels::matmul and its neighbours over the C-ABI. Host-side validation
// throws the reference's exception types before any device call
// (src/cuda/matmul.cu:132-137, src/cuda/embedding.cu:67-70,
// src/cuda/silu_multiply.cu:20); device-side failures arrive as C-ABI status
// codes and are rethrown (include/Kernels.hpp:28-32).
#include "Kernels.hpp"

#include <utility>

#include "qk_abi.h"

namespace kernels::detail {

void check_status(int status, const char* what) {
    if (status == QK_OK) return;
    const std::string message = std::string(what) + ": " + qk_last_error();
    if (status == QK_ERR_INVALID_ARGUMENT || status == QK_ERR_UNSUPPORTED_TYPE)
        throw std::invalid_argument(message);
    throw std::runtime_error(message);
}

void check_launch() { check_status(qk_check_launch(), "HIP kernel launch failed"); }

int get_sm_count() {
    int count = 0;
    check_status(qk_device_info(nullptr, 0, &count, nullptr, 0), "HIP device query failed");
    return count;
}

}  // namespace kernels::detail

namespace kernels {

using detail::check_status;

Stream::Stream() { check_status(qk_stream_create(&stream_), "HIP stream error"); }

Stream::~Stream() {
    if (stream_) qk_stream_destroy(stream_);
}

Stream::Stream(Stream&& other) noexcept : stream_(std::exchange(other.stream_, nullptr)) {}

Stream& Stream::operator=(Stream&& other) noexcept {
    if (this != &other) {
        if (stream_) qk_stream_destroy(stream_);
        stream_ = std::exchange(other.stream_, nullptr);
    }
    return *this;
}

stream_t Stream::get() const {
    if (!stream_) throw std::logic_error("HIP stream was moved from");
    return stream_;
}

void Stream::synchronize() const { check_status(qk_stream_synchronize(get()), "HIP stream error"); }

bool Stream::ready() const {
    int ready = 0;
    check_status(qk_stream_query(get(), &ready), "HIP stream error");
    return ready != 0;
}

void matmul(const float* input, const Weight& weight, float* output, size_t rows, stream_t stream) {
    if (weight.datatype != GGML_TYPE_Q4_K && weight.datatype != GGML_TYPE_Q6_K)
        throw std::invalid_argument("matmul supports Q4_K and Q6_K weights only");
    if (weight.dimension.size() < 2 || weight.dimension[0] <= 0 ||
        weight.dimension[0] % 256 != 0 || weight.dimension[1] <= 0)
        throw std::invalid_argument("Invalid matmul weight dimensions");
    if (rows == 0) return;
    check_status(qk_matmul(input, weight.device_buffer.data, weight.datatype, weight.dimension[0],
                           weight.dimension[1], output, static_cast<int64_t>(rows), stream),
                 "HIP kernel launch failed");
}

void matmul(const float* input, const Weight& weight, float* output, size_t rows, const Stream& stream) {
    matmul(input, weight, output, rows, stream.get());
}

void rms_norm(const float* input, const Weight& scale, float* output, size_t rows, size_t width,
              float epsilon) {
    if (rows == 0) return;  // src/cuda/rms_norm.cu:31-34
    if (width == 0 || !(epsilon > 0.0f) || scale.datatype != GGML_TYPE_F32 ||
        scale.dimension.empty() || static_cast<size_t>(scale.dimension[0]) != width)
        throw std::invalid_argument(
            "RMSNorm requires an F32 scale matching the row width and positive epsilon");
    check_status(qk_rms_norm(input, static_cast<const float*>(scale.device_buffer.data), output,
                             static_cast<int64_t>(rows), static_cast<int64_t>(width), epsilon,
                             nullptr),
                 "HIP kernel launch failed");
}

void residual_add(float* state, const float* branch, size_t count) {
    if (count == 0) return;  // src/cuda/residual_add.cu:16
    check_status(qk_residual_add(state, branch, static_cast<int64_t>(count), nullptr),
                 "HIP kernel launch failed");
}

void silu_multiply(const float* gate, const float* up, float* output, size_t count) {
    if (count == 0) return;
    check_status(qk_silu_multiply(gate, up, output, static_cast<int64_t>(count), nullptr),
                 "HIP kernel launch failed");
}

uint32_t argmax(const float* logits, size_t vocabulary_size) {
    if (!logits || vocabulary_size == 0 || vocabulary_size > UINT32_MAX)
        throw std::invalid_argument("Invalid argmax input");  // src/cuda/argmax.cu:73-74
    const size_t ws_bytes = qk_argmax_workspace_size();
    DeviceBuffer workspace(ws_bytes);
    DeviceBuffer result(sizeof(uint32_t));
    check_status(qk_memset_async(workspace.data, 0, ws_bytes, nullptr), "HIP memset failed");
    check_status(qk_argmax(logits, static_cast<int64_t>(vocabulary_size),
                           static_cast<uint32_t*>(result.data), workspace.data, ws_bytes, nullptr),
                 "HIP kernel launch failed");
    uint32_t index = 0;
    check_status(qk_memcpy_d2h(&index, result.data, sizeof(index), nullptr), "HIP copy failed");
    check_status(qk_argmax_workspace_check(workspace.data, nullptr), "HIP argmax failed");
    return index;
}

void dequantize_embeddings(const void* packed, float* output, size_t rows, size_t width,
                           size_t row_bytes, ggml_type type) {
    if (rows == 0) return;
    if (type != GGML_TYPE_Q4_K && type != GGML_TYPE_Q6_K)
        throw std::invalid_argument("Unsupported embedding storage type");
    check_status(qk_dequantize_rows(packed, output, static_cast<int64_t>(rows),
                                    static_cast<int64_t>(width), row_bytes, type, nullptr),
                 "HIP kernel launch failed");
}

}  // namespace kernels
