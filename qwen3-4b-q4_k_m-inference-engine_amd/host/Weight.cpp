// DeviceBuffer and Weight over the C-ABI memory shims (the reference's
// src/Weight.cpp:6-61 semantics: stream-ordered allocation, the host-to-device
// copy completes before the constructor returns, zero bytes hold nullptr).
#include "Weight.hpp"

#include <stdexcept>
#include <utility>

#include "GGUF.hpp"
#include "Kernels.hpp"
#include "qk_abi.h"

DeviceBuffer::DeviceBuffer(const void* source, std::size_t source_bytes, device_stream_t allocation_stream)
    : stream(allocation_stream) {
    if (source_bytes == 0) return;
    if (!source) throw std::invalid_argument("Nonempty DeviceBuffer requires host data");
    kernels::detail::check_status(qk_malloc_async(&data, source_bytes, stream), "qk_malloc_async failed");
    const int status = qk_memcpy_h2d(data, source, source_bytes, stream);
    if (status != QK_OK) {
        const std::string message = qk_last_error();
        qk_free_async(data, stream);
        data = nullptr;
        throw std::runtime_error("Host-to-device copy failed: " + message);
    }
    bytes = source_bytes;
}

DeviceBuffer::DeviceBuffer(std::size_t source_bytes, device_stream_t allocation_stream)
    : stream(allocation_stream) {
    if (source_bytes == 0) return;
    kernels::detail::check_status(qk_malloc_async(&data, source_bytes, stream), "qk_malloc_async failed");
    bytes = source_bytes;
}

DeviceBuffer::~DeviceBuffer() {
    if (data) qk_free_async(data, stream);
}

DeviceBuffer::DeviceBuffer(DeviceBuffer&& other) noexcept
    : data(std::exchange(other.data, nullptr)),
      bytes(std::exchange(other.bytes, 0)),
      stream(std::exchange(other.stream, nullptr)) {}

DeviceBuffer& DeviceBuffer::operator=(DeviceBuffer&& other) noexcept {
    if (this != &other) {
        if (data) qk_free_async(data, stream);
        data = std::exchange(other.data, nullptr);
        bytes = std::exchange(other.bytes, 0);
        stream = std::exchange(other.stream, nullptr);
    }
    return *this;
}

Weight::Weight(const GGUF& model, const std::string& tensor_name) : name(tensor_name) {
    const auto* tensor = model.get_tensor_info(name);
    datatype = tensor->type;
    dimension.assign(tensor->dimensions.begin(), tensor->dimensions.end());
    const auto data = model.read_tensor_data(name);
    // The kernels take the row count from dimension[1]: the bytes must hold
    // exactly every row of every plane.
    if (data.size() != gguf_tensor_bytes(datatype, tensor->dimensions))
        throw std::runtime_error("GGUF tensor size does not match its dimensions: " + name);
    device_buffer = DeviceBuffer(data.data(), data.size());
}

Weight::Weight(std::string tensor_name, ggml_type type, std::vector<std::int64_t> dims,
               const void* host_bytes, std::size_t size)
    : name(std::move(tensor_name)), datatype(type), dimension(std::move(dims)) {
    device_buffer = DeviceBuffer(host_bytes, size);
}
