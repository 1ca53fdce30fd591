// GGUF v2/v3 container reader (replaces the ggml gguf_* wrapper of the
// reference's src/GGUF.cpp:81-173). Layout: magic "GGUF", u32 version,
// u64 tensor count, u64 metadata count, metadata {string key, u32 type, value},
// tensor infos {string name, u32 n_dims, u64 ne[n_dims], u32 type, u64 offset},
// padding to general.alignment (default 32), then the data section.
#include "GGUF.hpp"

#include <algorithm>
#include <cstring>
#include <fstream>
#include <limits>
#include <stdexcept>

namespace {

struct TypeTraits {
    int64_t block;
    int64_t bytes;
};

// ggml block size / block bytes per type (ggml's type_traits table; file-format constants).
TypeTraits traits(ggml_type type) {
    switch (type) {
    case GGML_TYPE_F32: return {1, 4};
    case GGML_TYPE_F16: return {1, 2};
    case GGML_TYPE_BF16: return {1, 2};
    case GGML_TYPE_Q4_0: return {32, 18};
    case GGML_TYPE_Q4_1: return {32, 20};
    case GGML_TYPE_Q5_0: return {32, 22};
    case GGML_TYPE_Q5_1: return {32, 24};
    case GGML_TYPE_Q8_0: return {32, 34};
    case GGML_TYPE_Q8_1: return {32, 36};
    case GGML_TYPE_Q2_K: return {256, 84};
    case GGML_TYPE_Q3_K: return {256, 110};
    case GGML_TYPE_Q4_K: return {256, 144};
    case GGML_TYPE_Q5_K: return {256, 176};
    case GGML_TYPE_Q6_K: return {256, 210};
    case GGML_TYPE_Q8_K: return {256, 292};
    case GGML_TYPE_COUNT: break;
    }
    throw std::runtime_error("Unsupported GGUF tensor type " + std::to_string(int(type)));
}

class Reader {
public:
    explicit Reader(const std::filesystem::path& path) : file_(path, std::ios::binary) {
        if (!file_) throw std::runtime_error("Failed to read GGUF: " + path.string());
        file_.seekg(0, std::ios::end);
        size_ = static_cast<uint64_t>(file_.tellg());
        file_.seekg(0);
    }
    template <class T> T pod() {
        T v;
        bytes(&v, sizeof(T));
        return v;
    }
    void bytes(void* dst, size_t n) {
        if (n > size_ - pos_) throw std::runtime_error("Truncated GGUF file");
        file_.read(static_cast<char*>(dst), static_cast<std::streamsize>(n));
        if (!file_) throw std::runtime_error("Truncated GGUF file");
        pos_ += n;
    }
    std::string string() {
        const uint64_t n = pod<uint64_t>();
        if (n > size_ - pos_) throw std::runtime_error("Truncated GGUF string");
        std::string s(n, '\0');
        bytes(s.data(), n);
        return s;
    }
    uint64_t pos() const { return pos_; }
    uint64_t size() const { return size_; }

private:
    std::ifstream file_;
    uint64_t size_{0};
    uint64_t pos_{0};
};

template <class T> std::vector<T> read_array(Reader& in, uint64_t count) {
    if (count > in.size()) throw std::runtime_error("Truncated GGUF array");
    std::vector<T> out;
    out.reserve(count);
    for (uint64_t i = 0; i < count; ++i) {
        if constexpr (std::is_same_v<T, std::string>)
            out.push_back(in.string());
        else if constexpr (std::is_same_v<T, bool>)
            out.push_back(in.pod<int8_t>() != 0);
        else
            out.push_back(in.pod<T>());
    }
    return out;
}

GGUF::MetadataValue read_scalar(Reader& in, gguf_type type) {
    switch (type) {
    case GGUF_TYPE_UINT8: return in.pod<uint8_t>();
    case GGUF_TYPE_INT8: return in.pod<int8_t>();
    case GGUF_TYPE_UINT16: return in.pod<uint16_t>();
    case GGUF_TYPE_INT16: return in.pod<int16_t>();
    case GGUF_TYPE_UINT32: return in.pod<uint32_t>();
    case GGUF_TYPE_INT32: return in.pod<int32_t>();
    case GGUF_TYPE_FLOAT32: return in.pod<float>();
    case GGUF_TYPE_BOOL: return in.pod<int8_t>() != 0;
    case GGUF_TYPE_STRING: return in.string();
    case GGUF_TYPE_UINT64: return in.pod<uint64_t>();
    case GGUF_TYPE_INT64: return in.pod<int64_t>();
    case GGUF_TYPE_FLOAT64: return in.pod<double>();
    default: throw std::runtime_error("Unsupported GGUF scalar type");
    }
}

GGUF::MetadataValue read_array_value(Reader& in, gguf_type type, uint64_t count) {
    switch (type) {
    case GGUF_TYPE_UINT8: return read_array<uint8_t>(in, count);
    case GGUF_TYPE_INT8: return read_array<int8_t>(in, count);
    case GGUF_TYPE_UINT16: return read_array<uint16_t>(in, count);
    case GGUF_TYPE_INT16: return read_array<int16_t>(in, count);
    case GGUF_TYPE_UINT32: return read_array<uint32_t>(in, count);
    case GGUF_TYPE_INT32: return read_array<int32_t>(in, count);
    case GGUF_TYPE_FLOAT32: return read_array<float>(in, count);
    case GGUF_TYPE_BOOL: return read_array<bool>(in, count);
    case GGUF_TYPE_STRING: return read_array<std::string>(in, count);
    case GGUF_TYPE_UINT64: return read_array<uint64_t>(in, count);
    case GGUF_TYPE_INT64: return read_array<int64_t>(in, count);
    case GGUF_TYPE_FLOAT64: return read_array<double>(in, count);
    default: throw std::runtime_error("Unsupported GGUF array element type");
    }
}

}  // namespace

// Bytes of a tensor of `type` with ggml dimensions ne (each >= 1). Every
// product is checked: a corrupt header whose element count or byte size
// exceeds INT64_MAX is rejected rather than wrapped to a small size that
// would pass the bounds checks.
std::size_t gguf_tensor_bytes(ggml_type type, const std::array<int64_t, GGUF_MAX_DIMS>& ne) {
    const TypeTraits t = traits(type);
    for (int i = 0; i < GGUF_MAX_DIMS; ++i)
        if (ne[i] <= 0) throw std::runtime_error("GGUF tensor dimension must be positive");
    if (ne[0] % t.block != 0) throw std::runtime_error("GGUF row width is not a whole number of blocks");
    int64_t elements = ne[0], bytes = 0;
    for (int i = 1; i < GGUF_MAX_DIMS; ++i)
        if (__builtin_mul_overflow(elements, ne[i], &elements))
            throw std::runtime_error("GGUF tensor element count overflows");
    int64_t rows = 1;
    for (int i = 1; i < GGUF_MAX_DIMS; ++i) rows *= ne[i];  // <= elements: no overflow
    if (__builtin_mul_overflow(ne[0] / t.block * t.bytes, rows, &bytes) ||
        static_cast<uint64_t>(bytes) > std::numeric_limits<std::size_t>::max())
        throw std::runtime_error("GGUF tensor byte size overflows");
    return static_cast<std::size_t>(bytes);
}

GGUF::GGUF(const std::filesystem::path& path, bool load_weights) : path_(path) {
    Reader in(path_);
    char magic[4];
    in.bytes(magic, 4);
    if (std::memcmp(magic, "GGUF", 4) != 0) throw std::runtime_error("Not a GGUF file: " + path_.string());
    version_ = in.pod<uint32_t>();
    if (version_ < 2 || version_ > 3) throw std::runtime_error("Unsupported GGUF version");
    const uint64_t n_tensors = in.pod<uint64_t>();
    const uint64_t n_kv = in.pod<uint64_t>();
    if (n_tensors > in.size() || n_kv > in.size()) throw std::runtime_error("Corrupt GGUF header");

    for (uint64_t i = 0; i < n_kv; ++i) {
        std::string key = in.string();
        const auto type = static_cast<gguf_type>(in.pod<uint32_t>());
        Metadata entry{type, std::nullopt, uint8_t{0}};
        if (type == GGUF_TYPE_ARRAY) {
            const auto element = static_cast<gguf_type>(in.pod<uint32_t>());
            const uint64_t count = in.pod<uint64_t>();
            entry.element_type = element;
            entry.value = read_array_value(in, element, count);
        } else {
            entry.value = read_scalar(in, type);
        }
        metadata_.emplace(std::move(key), std::move(entry));
    }
    if (auto a = get_value<uint32_t>("general.alignment")) alignment_ = *a;
    if (alignment_ == 0 || (alignment_ & (alignment_ - 1)) != 0)
        throw std::runtime_error("GGUF alignment must be a power of two");

    std::vector<uint64_t> offsets;
    for (uint64_t i = 0; i < n_tensors; ++i) {
        TensorInfo info{};
        info.name = in.string();
        const uint32_t n_dims = in.pod<uint32_t>();
        if (n_dims > GGUF_MAX_DIMS) throw std::runtime_error("GGUF tensor has too many dimensions");
        info.dimensions = {1, 1, 1, 1};
        for (uint32_t d = 0; d < n_dims; ++d) {
            const auto ne = in.pod<int64_t>();
            if (ne <= 0) throw std::runtime_error("GGUF tensor dimension must be positive");
            info.dimensions[d] = ne;
        }
        info.type = static_cast<ggml_type>(in.pod<uint32_t>());
        offsets.push_back(in.pod<uint64_t>());
        info.bytes = gguf_tensor_bytes(info.type, info.dimensions);
        tensors_.push_back(std::move(info));
    }
    data_offset_ = (in.pos() + alignment_ - 1) / alignment_ * alignment_;
    // A file with tensors must hold its whole data section; one without may
    // end before the padding.
    if (!tensors_.empty() && data_offset_ > in.size())
        throw std::runtime_error("Incomplete GGUF data section");
    for (size_t i = 0; i < tensors_.size(); ++i) {
        if (offsets[i] % alignment_ != 0)
            throw std::runtime_error("GGUF tensor data is not aligned: " + tensors_[i].name);
        if (offsets[i] > in.size() - data_offset_ ||
            tensors_[i].bytes > in.size() - data_offset_ - offsets[i])
            throw std::runtime_error("Incomplete GGUF tensor data: " + tensors_[i].name);
        tensors_[i].file_offset = data_offset_ + offsets[i];
    }
    if (load_weights) {
        std::ifstream file(path_, std::ios::binary);
        file.seekg(static_cast<std::streamoff>(std::min(data_offset_, in.size())));
        weights_.resize(data_offset_ < in.size() ? in.size() - data_offset_ : 0);
        if (!file.read(reinterpret_cast<char*>(weights_.data()), static_cast<std::streamsize>(weights_.size())))
            throw std::runtime_error("Failed to read GGUF data section");
    }
}

const GGUF::Metadata* GGUF::get_metadata(const std::string& key) const {
    const auto it = metadata_.find(key);
    return it == metadata_.end() ? nullptr : &it->second;
}

const GGUF::TensorInfo* GGUF::get_tensor_info(const std::string& name) const {
    const auto it = std::find_if(tensors_.begin(), tensors_.end(),
        [&](const TensorInfo& tensor) { return tensor.name == name; });
    if (it == tensors_.end()) throw std::runtime_error("Tensor unavailable: " + name);
    return &*it;
}

std::span<const std::byte> GGUF::get_tensor_data(const std::string& name) const {
    if (weights_.empty()) throw std::logic_error("Construct GGUF with load_weights=true to access weights");
    const auto it = std::find_if(tensors_.begin(), tensors_.end(),
        [&](const TensorInfo& tensor) { return tensor.name == name; });
    if (it == tensors_.end()) throw std::out_of_range("Unknown tensor: " + name);
    return {weights_.data() + (it->file_offset - data_offset_), it->bytes};
}

std::vector<std::byte> GGUF::read_tensor_data(const std::string& name) const {
    const auto* info = get_tensor_info(name);
    std::ifstream file(path_, std::ios::binary | std::ios::ate);
    if (!file) throw std::runtime_error("Failed to open GGUF: " + path_.string());
    const auto end = file.tellg();
    if (end < 0 || info->file_offset > static_cast<uint64_t>(end) ||
        info->bytes > static_cast<uint64_t>(end) - info->file_offset)
        throw std::runtime_error("Incomplete GGUF tensor data: " + name);
    file.seekg(static_cast<std::streamoff>(info->file_offset));
    std::vector<std::byte> data(info->bytes);
    if (!file.read(reinterpret_cast<char*>(data.data()), static_cast<std::streamsize>(data.size())))
        throw std::runtime_error("Failed to read tensor: " + name);
    return data;
}

std::optional<uint32_t> GGUF::architecture_value(const std::string& suffix) const {
    const auto arch = get_architecture();
    return arch ? get_value<uint32_t>(*arch + "." + suffix) : std::nullopt;
}
std::optional<std::string> GGUF::get_name() const { return get_value<std::string>("general.name"); }
std::optional<std::string> GGUF::get_architecture() const { return get_value<std::string>("general.architecture"); }
std::optional<uint32_t> GGUF::get_context_length() const { return architecture_value("context_length"); }
std::optional<uint32_t> GGUF::get_embedding_length() const { return architecture_value("embedding_length"); }
std::optional<uint32_t> GGUF::get_layer_count() const { return architecture_value("block_count"); }
std::optional<uint32_t> GGUF::get_attention_head_count() const { return architecture_value("attention.head_count"); }

void GGUF::free_weights() {
    weights_.clear();
    weights_.shrink_to_fit();
}
