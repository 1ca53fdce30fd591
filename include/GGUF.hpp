#pragma once
// GGUF metadata and tensor-info reader with the interface of the reference's
// include/GGUF.hpp:17-135, parsing the GGUF v2/v3 container itself instead of
// wrapping ggml's gguf_* (src/GGUF.cpp:81-111). Tensor data are read per tensor
// from the file (src/GGUF.cpp:131-145) or, optionally, loaded whole into RAM.
#include <array>
#include <cstddef>
#include <cstdint>
#include <filesystem>
#include <map>
#include <optional>
#include <span>
#include <string>
#include <variant>
#include <vector>

#include "ggml_type.hpp"

// GGUF metadata value types (the container's on-disk ids).
enum gguf_type : uint32_t {
    GGUF_TYPE_UINT8 = 0,
    GGUF_TYPE_INT8 = 1,
    GGUF_TYPE_UINT16 = 2,
    GGUF_TYPE_INT16 = 3,
    GGUF_TYPE_UINT32 = 4,
    GGUF_TYPE_INT32 = 5,
    GGUF_TYPE_FLOAT32 = 6,
    GGUF_TYPE_BOOL = 7,
    GGUF_TYPE_STRING = 8,
    GGUF_TYPE_ARRAY = 9,
    GGUF_TYPE_UINT64 = 10,
    GGUF_TYPE_INT64 = 11,
    GGUF_TYPE_FLOAT64 = 12,
};

inline constexpr int GGUF_MAX_DIMS = 4;

// Bytes of a tensor of the given type and ne[] (throws for unknown types).
std::size_t gguf_tensor_bytes(ggml_type type, const std::array<int64_t, GGUF_MAX_DIMS>& ne);

class GGUF {
public:
    using MetadataValue = std::variant<
        uint8_t, int8_t, uint16_t, int16_t, uint32_t, int32_t,
        float, bool, std::string, uint64_t, int64_t, double,
        std::vector<uint8_t>, std::vector<int8_t>, std::vector<uint16_t>,
        std::vector<int16_t>, std::vector<uint32_t>, std::vector<int32_t>,
        std::vector<float>, std::vector<bool>, std::vector<std::string>,
        std::vector<uint64_t>, std::vector<int64_t>, std::vector<double>>;
    struct Metadata {
        gguf_type type;
        std::optional<gguf_type> element_type;  // arrays only
        MetadataValue value;
    };
    struct TensorInfo {
        std::string name;
        std::array<int64_t, GGUF_MAX_DIMS> dimensions;  // unused axes are 1
        ggml_type type;
        size_t bytes;
        size_t file_offset;  // absolute offset in the file
    };

    // Parses the header; load_weights=true also reads all tensor data into RAM.
    // Throws std::runtime_error on a malformed or truncated file.
    explicit GGUF(const std::filesystem::path& path, bool load_weights = false);
    GGUF(const GGUF&) = delete;
    GGUF& operator=(const GGUF&) = delete;

    const std::filesystem::path& get_path() const { return path_; }
    uint32_t get_version() const { return version_; }
    size_t get_alignment() const { return alignment_; }
    size_t get_data_offset() const { return data_offset_; }
    bool has_weights() const { return !weights_.empty(); }

    const std::map<std::string, Metadata>& get_metadata() const { return metadata_; }
    const Metadata* get_metadata(const std::string& key) const;
    const std::vector<TensorInfo>& get_tensors() const { return tensors_; }
    // Throws std::runtime_error if absent.
    const TensorInfo* get_tensor_info(const std::string& name) const;
    // Borrowed bytes of a loaded tensor; throws if weights were not loaded or name is absent.
    std::span<const std::byte> get_tensor_data(const std::string& name) const;
    // Reads one tensor from disk; the caller owns the buffer.
    std::vector<std::byte> read_tensor_data(const std::string& name) const;

    template <class T> std::optional<T> get_value(const std::string& key) const {
        const auto* entry = get_metadata(key);
        if (!entry) return std::nullopt;
        const auto* value = std::get_if<T>(&entry->value);
        return value ? std::optional<T>(*value) : std::nullopt;
    }
    template <class T> const std::vector<T>* get_array(const std::string& key) const {
        const auto* entry = get_metadata(key);
        return entry ? std::get_if<std::vector<T>>(&entry->value) : nullptr;
    }

    std::optional<std::string> get_name() const;
    std::optional<std::string> get_architecture() const;
    std::optional<uint32_t> get_context_length() const;
    std::optional<uint32_t> get_embedding_length() const;
    std::optional<uint32_t> get_layer_count() const;
    std::optional<uint32_t> get_attention_head_count() const;

    void free_weights();

private:
    std::optional<uint32_t> architecture_value(const std::string& suffix) const;

    std::filesystem::path path_;
    uint32_t version_{0};
    size_t alignment_{32};
    size_t data_offset_{0};
    std::map<std::string, Metadata> metadata_;
    std::vector<TensorInfo> tensors_;
    std::vector<std::byte> weights_;  // whole data section when loaded
};
