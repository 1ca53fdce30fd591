// EmbedLookup over this repository's GGUF reader and kernels (the reference's
// src/EmbedLookup.cpp:11-78 contract: validation order, exception types,
// empty lookups, rows in input order).
#include "EmbedLookup.hpp"

#include <cstring>
#include <stdexcept>
#include <utility>

#include "Kernels.hpp"

EmbedLookup::EmbedLookup(const GGUF& model, const std::string& tensor_name) {
    const GGUF::TensorInfo* info = model.get_tensor_info(tensor_name);
    const auto& ne = info->dimensions;
    type_ = info->type;
    const std::array<int64_t, GGUF_MAX_DIMS> one_row{ne[0], 1, 1, 1};
    size_t row_bytes = 0;
    try {
        // throws for a type it does not know or a width that is not whole blocks
        row_bytes = ne[0] > 0 ? gguf_tensor_bytes(type_, one_row) : 0;
    } catch (const std::runtime_error&) {
        row_bytes = 0;
    }
    if (row_bytes == 0 || ne[1] <= 0 || ne[2] != 1 || ne[3] != 1)
        throw std::invalid_argument("Invalid embedding dimensions for tensor storage type");
    width_ = static_cast<size_t>(ne[0]);
    vocabulary_ = static_cast<size_t>(ne[1]);
    row_bytes_ = row_bytes;
    if (info->bytes / row_bytes_ != vocabulary_ || info->bytes % row_bytes_ != 0)
        throw std::invalid_argument("Embedding tensor byte size does not match its dimensions");
    table_ = model.read_tensor_data(tensor_name);
}

EmbedLookup::EmbedLookup(EmbedLookup&& other) noexcept
    : type_(std::exchange(other.type_, GGML_TYPE_COUNT)),
      table_(std::move(other.table_)),
      width_(std::exchange(other.width_, 0)),
      vocabulary_(std::exchange(other.vocabulary_, 0)),
      row_bytes_(std::exchange(other.row_bytes_, 0)) {}

EmbedLookup& EmbedLookup::operator=(EmbedLookup&& other) noexcept {
    if (this != &other) {
        type_ = std::exchange(other.type_, GGML_TYPE_COUNT);
        table_ = std::move(other.table_);
        width_ = std::exchange(other.width_, 0);
        vocabulary_ = std::exchange(other.vocabulary_, 0);
        row_bytes_ = std::exchange(other.row_bytes_, 0);
    }
    return *this;
}

DeviceBuffer EmbedLookup::lookup(const std::vector<uint32_t>& token_ids) const {
    for (const uint32_t id : token_ids)
        if (id >= vocabulary_) throw std::out_of_range("Embedding token ID out of range");
    if (type_ != GGML_TYPE_F32 && type_ != GGML_TYPE_Q4_K && type_ != GGML_TYPE_Q6_K)
        throw std::invalid_argument("Unsupported embedding storage type");
    if (token_ids.empty()) return DeviceBuffer(size_t{0});

    // Only the requested rows cross PCIe, packed back to back in input order.
    std::vector<std::byte> gathered(token_ids.size() * row_bytes_);
    std::byte* dst = gathered.data();
    for (const uint32_t id : token_ids) {
        std::memcpy(dst, table_.data() + static_cast<size_t>(id) * row_bytes_, row_bytes_);
        dst += row_bytes_;
    }
    DeviceBuffer rows(gathered.data(), gathered.size());
    if (type_ == GGML_TYPE_F32) return rows;
    DeviceBuffer out(token_ids.size() * width_ * sizeof(float));
    kernels::dequantize_embeddings(rows.data, static_cast<float*>(out.data), token_ids.size(), width_,
                                   row_bytes_, type_);
    return out;
}
