// CPU-only tests of the C++ host layer: the argument validation of
// kernels::matmul / dequantize_embeddings (src/cuda/matmul.cu:132-137,
// src/cuda/embedding.cu:67-70), empty DeviceBuffers (src/Weight.cpp:8,27), the
// status -> exception mapping, and the GGUF reader on a file written here.
// Nothing in this binary touches a device: every call below returns or
// throws before the C-ABI reaches HIP.
#include <cmath>
#include <cstdint>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <limits>
#include <stdexcept>
#include <vector>

#include "GGUF.hpp"
#include "Kernels.hpp"
#include "Weight.hpp"
#include "mini_test.hpp"
#include "qk_abi.h"

namespace {

Weight empty_weight(ggml_type type, std::vector<int64_t> dims) {
    return Weight("blk.0.test.weight", type, std::move(dims), nullptr, 0);
}

}  // namespace

TEST_CASE("empty DeviceBuffer holds nullptr and zero bytes") {
    DeviceBuffer a(nullptr, 0);
    REQUIRE(a.data == nullptr && a.bytes == 0);
    DeviceBuffer b(std::size_t{0});
    REQUIRE(b.data == nullptr && b.bytes == 0);
    DeviceBuffer c(std::move(a));
    REQUIRE(c.data == nullptr && c.bytes == 0);
    REQUIRE_THROWS_AS(DeviceBuffer(nullptr, 16), std::invalid_argument);
}

TEST_CASE("matmul rejects unsupported weight types") {
    float x = 0, y = 0;
    for (auto type : {GGML_TYPE_F32, GGML_TYPE_F16, GGML_TYPE_Q4_0, GGML_TYPE_Q5_K, GGML_TYPE_Q8_0}) {
        const Weight w = empty_weight(type, {2560, 8});
        REQUIRE_THROWS_AS(kernels::matmul(&x, w, &y, 1), std::invalid_argument);
    }
}

TEST_CASE("matmul rejects invalid dimensions") {
    float x = 0, y = 0;
    for (auto dims : std::vector<std::vector<int64_t>>{{2560}, {2500, 8}, {0, 8}, {-256, 8},
                                                        {2560, 0}, {2560, -1}, {}}) {
        const Weight w = empty_weight(GGML_TYPE_Q4_K, dims);
        REQUIRE_THROWS_AS(kernels::matmul(&x, w, &y, 1), std::invalid_argument);
    }
}

TEST_CASE("matmul with zero rows returns without launching") {
    const Weight q4 = empty_weight(GGML_TYPE_Q4_K, {2560, 8});
    const Weight q6 = empty_weight(GGML_TYPE_Q6_K, {9728, 8, 1, 1});
    REQUIRE_NOTHROW(kernels::matmul(nullptr, q4, nullptr, 0));
    REQUIRE_NOTHROW(kernels::matmul(nullptr, q6, nullptr, 0));
}

TEST_CASE("dequantize_embeddings validation") {
    REQUIRE_NOTHROW(kernels::dequantize_embeddings(nullptr, nullptr, 0, 2560, 1440, GGML_TYPE_F32));
    REQUIRE_THROWS_AS(kernels::dequantize_embeddings(nullptr, nullptr, 1, 2560, 1440, GGML_TYPE_F32),
                      std::invalid_argument);
    REQUIRE_NOTHROW(kernels::silu_multiply(nullptr, nullptr, nullptr, 0));
}

TEST_CASE("argmax rejects invalid input before touching the device") {
    float x = 0;
    REQUIRE_THROWS_AS(kernels::argmax(nullptr, 5), std::invalid_argument);  // argmax.cu:73-74
    REQUIRE_THROWS_AS(kernels::argmax(&x, 0), std::invalid_argument);
    REQUIRE_THROWS_AS(kernels::argmax(&x, size_t{UINT32_MAX} + 1), std::invalid_argument);
}

TEST_CASE("C-ABI status maps to the reference's exception types") {
    REQUIRE_NOTHROW(kernels::detail::check_status(QK_OK, "ok"));
    REQUIRE_THROWS_AS(kernels::detail::check_status(QK_ERR_INVALID_ARGUMENT, "x"), std::invalid_argument);
    REQUIRE_THROWS_AS(kernels::detail::check_status(QK_ERR_UNSUPPORTED_TYPE, "x"), std::invalid_argument);
    REQUIRE_THROWS_AS(kernels::detail::check_status(QK_ERR_RUNTIME, "x"), std::runtime_error);
    REQUIRE_THROWS_AS(kernels::detail::check_status(QK_ERR_OUT_OF_MEMORY, "x"), std::runtime_error);
}

namespace {

struct GgufWriter {
    std::vector<unsigned char> out;
    template <class T> void pod(T v) {
        const auto* p = reinterpret_cast<const unsigned char*>(&v);
        out.insert(out.end(), p, p + sizeof(T));
    }
    void str(const std::string& s) {
        pod<uint64_t>(s.size());
        out.insert(out.end(), s.begin(), s.end());
    }
};

}  // namespace

TEST_CASE("GGUF reader parses metadata, tensor infos and data") {
    // two tensors: a Q4_K [512 x 3] and an F32 [7]
    GgufWriter w;
    w.out.insert(w.out.end(), {'G', 'G', 'U', 'F'});
    w.pod<uint32_t>(3);
    w.pod<uint64_t>(2);  // tensors
    w.pod<uint64_t>(4);  // kv
    w.str("general.architecture"); w.pod<uint32_t>(GGUF_TYPE_STRING); w.str("qwen3");
    w.str("qwen3.block_count"); w.pod<uint32_t>(GGUF_TYPE_UINT32); w.pod<uint32_t>(36);
    w.str("general.alignment"); w.pod<uint32_t>(GGUF_TYPE_UINT32); w.pod<uint32_t>(64);
    w.str("tokenizer.ggml.scores"); w.pod<uint32_t>(GGUF_TYPE_ARRAY); w.pod<uint32_t>(GGUF_TYPE_FLOAT32);
    w.pod<uint64_t>(3); w.pod<float>(0.5f); w.pod<float>(-1.0f); w.pod<float>(2.0f);
    w.str("blk.0.ffn_gate.weight"); w.pod<uint32_t>(2); w.pod<int64_t>(512); w.pod<int64_t>(3);
    w.pod<uint32_t>(GGML_TYPE_Q4_K); w.pod<uint64_t>(0);
    w.str("output_norm.weight"); w.pod<uint32_t>(1); w.pod<int64_t>(7);
    w.pod<uint32_t>(GGML_TYPE_F32); w.pod<uint64_t>(896);
    while (w.out.size() % 64) w.out.push_back(0);
    const size_t data_start = w.out.size();
    for (size_t i = 0; i < 896; ++i) w.out.push_back(static_cast<unsigned char>(i * 7));
    for (int i = 0; i < 7; ++i) w.pod<float>(float(i) * 0.25f);

    const auto path = std::filesystem::temp_directory_path() / "qk_host_test.gguf";
    {
        std::ofstream f(path, std::ios::binary);
        f.write(reinterpret_cast<const char*>(w.out.data()), static_cast<std::streamsize>(w.out.size()));
    }
    const GGUF model(path, true);
    REQUIRE(model.get_version() == 3);
    REQUIRE(model.get_alignment() == 64);
    REQUIRE(model.get_data_offset() == data_start);
    REQUIRE(model.get_architecture().value() == "qwen3");
    REQUIRE(model.get_layer_count().value() == 36);
    REQUIRE(model.get_array<float>("tokenizer.ggml.scores")->at(1) == -1.0f);
    REQUIRE(!model.get_value<float>("qwen3.block_count").has_value());
    const auto* info = model.get_tensor_info("blk.0.ffn_gate.weight");
    REQUIRE(info->type == GGML_TYPE_Q4_K && info->bytes == 3 * 288);
    REQUIRE(info->dimensions[0] == 512 && info->dimensions[1] == 3 && info->dimensions[2] == 1);
    const auto data = model.read_tensor_data("blk.0.ffn_gate.weight");
    REQUIRE(data.size() == 864 && std::to_integer<int>(data[5]) == 35);
    const auto norm = model.get_tensor_data("output_norm.weight");
    float v;
    std::memcpy(&v, norm.data() + 12, 4);
    REQUIRE(v == 0.75f);
    REQUIRE_THROWS_AS(model.get_tensor_info("missing"), std::runtime_error);
    std::filesystem::remove(path);

    const auto bad = std::filesystem::temp_directory_path() / "qk_host_test_bad.gguf";
    {
        std::ofstream f(bad, std::ios::binary);
        f.write(reinterpret_cast<const char*>(w.out.data()), 40);  // truncated header
    }
    REQUIRE_THROWS_AS(GGUF{bad}, std::runtime_error);
    std::filesystem::remove(bad);
}

namespace {

std::filesystem::path write_file(const char* name, const std::vector<unsigned char>& bytes) {
    const auto path = std::filesystem::temp_directory_path() / name;
    std::ofstream f(path, std::ios::binary);
    f.write(reinterpret_cast<const char*>(bytes.data()), static_cast<std::streamsize>(bytes.size()));
    return path;
}

GgufWriter header(uint64_t tensors) {
    GgufWriter w;
    w.out.insert(w.out.end(), {'G', 'G', 'U', 'F'});
    w.pod<uint32_t>(3);
    w.pod<uint64_t>(tensors);
    w.pod<uint64_t>(0);  // no metadata: alignment 32
    return w;
}

}  // namespace

TEST_CASE("GGUF reader rejects a tensor whose byte size wraps") {
    // ne = [256, 2^20, 2^22, 2^22]: 2^72 weights; 144 * 2^64 bytes wraps to 0 in 64 bits
    GgufWriter w = header(1);
    w.str("blk.0.wrapped.weight");
    w.pod<uint32_t>(4);
    for (int64_t ne : {int64_t{256}, int64_t{1} << 20, int64_t{1} << 22, int64_t{1} << 22}) w.pod<int64_t>(ne);
    w.pod<uint32_t>(GGML_TYPE_Q4_K);
    w.pod<uint64_t>(0);
    while (w.out.size() % 32) w.out.push_back(0);
    w.out.resize(w.out.size() + 144, 0);
    const auto path = write_file("qk_host_test_wrap.gguf", w.out);
    REQUIRE_THROWS_AS(GGUF{path}, std::runtime_error);
    std::filesystem::remove(path);
    std::array<int64_t, GGUF_MAX_DIMS> ne{256, int64_t{1} << 20, int64_t{1} << 22, int64_t{1} << 22};
    REQUIRE_THROWS_AS(gguf_tensor_bytes(GGML_TYPE_Q4_K, ne), std::runtime_error);
    ne = {2560, 9728, 1, 1};
    REQUIRE(gguf_tensor_bytes(GGML_TYPE_Q4_K, ne) == std::size_t{9728} * 10 * 144);
}

TEST_CASE("GGUF reader takes a header-only file and rejects a misaligned tensor") {
    // no tensors and no data padding: the data section is empty, not negative
    GgufWriter w = header(0);
    const auto path = write_file("qk_host_test_empty.gguf", w.out);
    const GGUF model(path, true);
    REQUIRE(model.get_tensors().empty());
    REQUIRE(!model.has_weights());
    std::filesystem::remove(path);

    GgufWriter m = header(1);
    m.str("blk.0.ffn_gate.weight");
    m.pod<uint32_t>(2);
    m.pod<int64_t>(256);
    m.pod<int64_t>(1);
    m.pod<uint32_t>(GGML_TYPE_Q4_K);
    m.pod<uint64_t>(16);  // not a multiple of the 32-byte alignment
    while (m.out.size() % 32) m.out.push_back(0);
    m.out.resize(m.out.size() + 16 + 144, 0);
    const auto bad = write_file("qk_host_test_misaligned.gguf", m.out);
    REQUIRE_THROWS_AS(GGUF{bad}, std::runtime_error);
    std::filesystem::remove(bad);

    GgufWriter t = header(1);  // a tensor but the file ends inside the header padding
    t.str("x");
    t.pod<uint32_t>(1);
    t.pod<int64_t>(256);
    t.pod<uint32_t>(GGML_TYPE_Q4_K);
    t.pod<uint64_t>(0);
    const auto cut = write_file("qk_host_test_cut.gguf", t.out);
    REQUIRE_THROWS_AS(GGUF{cut}, std::runtime_error);
    std::filesystem::remove(cut);
}

int main() { return mini::run_all(); }
