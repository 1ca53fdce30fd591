#pragma once
// Token embedding table kept on the host in its GGUF storage format, with the
// interface of the reference's include/EmbedLookup.hpp:9-33. lookup() gathers
// the requested rows on the host, uploads only those and dequantizes them on
// the device through kernels::dequantize_embeddings (the dequant core of the
// Q4_K/Q6_K path); F32 rows are returned as uploaded.
#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

#include "GGUF.hpp"
#include "Weight.hpp"

class EmbedLookup {
public:
    // Throws std::invalid_argument unless the tensor is [width x vocabulary]
    // (ne[2] = ne[3] = 1) with width a whole number of its type's blocks and
    // its byte size matching (src/EmbedLookup.cpp:11-28).
    explicit EmbedLookup(const GGUF& model, const std::string& tensor_name = "token_embd.weight");
    EmbedLookup(const EmbedLookup&) = delete;
    EmbedLookup& operator=(const EmbedLookup&) = delete;
    EmbedLookup(EmbedLookup&& other) noexcept;
    EmbedLookup& operator=(EmbedLookup&& other) noexcept;

    // fp32 [token_ids.size() x get_embedding_size()] on the device, one row per
    // id in input order. Throws std::out_of_range for an id >= vocabulary size
    // and std::invalid_argument for a table that is not F32, Q4_K or Q6_K; an
    // empty id list gives an empty buffer (src/EmbedLookup.cpp:49-78).
    DeviceBuffer lookup(const std::vector<uint32_t>& token_ids) const;
    size_t get_embedding_size() const { return width_; }
    size_t get_vocabulary_size() const { return vocabulary_; }
    ggml_type get_type() const { return type_; }
    size_t get_row_bytes() const { return row_bytes_; }

private:
    ggml_type type_{GGML_TYPE_COUNT};
    std::vector<std::byte> table_;
    size_t width_{0};
    size_t vocabulary_{0};
    size_t row_bytes_{0};
};
