#pragma once
// Device memory ownership and GGUF tensors on the device, with the interface
// of the reference's include/Weight.hpp:8-31. No HIP header is included: the
// stream is an opaque handle and every device call goes through the C-ABI
// (include/qk_abi.h).
#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

#include "ggml_type.hpp"

// Opaque device stream (a hipStream_t); nullptr is the null stream.
using device_stream_t = void*;

// RAII, move-only, stream-ordered device allocation
// (include/Weight.hpp:8-23, src/Weight.cpp:6-51). Zero bytes hold nullptr.
struct DeviceBuffer {
    void* data{nullptr};
    std::size_t bytes{0};

    device_stream_t stream{nullptr};

    // Allocates and copies `bytes` from host memory; returns once the copy is done.
    DeviceBuffer(const void* source, std::size_t bytes, device_stream_t stream = nullptr);
    explicit DeviceBuffer(std::size_t bytes, device_stream_t stream = nullptr);
    ~DeviceBuffer();

    DeviceBuffer(const DeviceBuffer& other) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;

    DeviceBuffer(DeviceBuffer&& other) noexcept;
    DeviceBuffer& operator=(DeviceBuffer&& other) noexcept;
};

class GGUF;

// A GGUF tensor's raw bytes on the device, copied verbatim (no repacking),
// plus its name, type and ggml ne[] dimensions: dimension[0] is the
// contiguous width K, dimension[1] the row count N (include/Weight.hpp:25-31).
struct Weight {
    std::string name;
    ggml_type datatype;
    DeviceBuffer device_buffer{nullptr, 0};
    std::vector<std::int64_t> dimension;

    // Reads the tensor from a GGUF file (src/Weight.cpp:53-61).
    Weight(const GGUF& model, const std::string& name);
    // Uploads a tensor from host bytes, e.g. synthetic superblocks.
    Weight(std::string name, ggml_type datatype, std::vector<std::int64_t> dimension,
           const void* host_bytes, std::size_t bytes);
};
