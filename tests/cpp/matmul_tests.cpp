// GPU test of the C++ host layer, mirroring src/tests/MatmulTests.cpp on
// synthetic superblocks (the reference reads blk.0.attn_q / attn_v / ffn_down
// from the model file, which is absent here): same shapes per type, same
// Approx criterion, overwrite on reuse, two non-blocking streams, sentinels
// around an offset output, zero input -> exact zeros. The expected values come
// from the CPU oracle (oracle/qk_oracle.c).
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <limits>
#include <vector>

#include "EmbedLookup.hpp"
#include "GGUF.hpp"
#include "Kernels.hpp"
#include "Weight.hpp"
#include "mini_test.hpp"
#include "qk_abi.h"
#include "qk_oracle.h"

namespace {

struct Tensor {
    const char* name;
    ggml_type type;
    int64_t width;
    int64_t rows;
};

// Qwen3-4B: attn_q Q4_K 2560 -> 4096, attn_v Q6_K 2560 -> 1024, ffn_down Q6_K 9728 -> 2560
const Tensor kTensors[] = {
    {"blk.0.attn_q.weight", GGML_TYPE_Q4_K, 2560, 4096},
    {"blk.0.attn_v.weight", GGML_TYPE_Q6_K, 2560, 1024},
    {"blk.0.ffn_down.weight", GGML_TYPE_Q6_K, 9728, 2560},
};

std::vector<unsigned char> synth(const Tensor& t, uint64_t seed) {
    std::vector<unsigned char> bytes(static_cast<size_t>(ggml_row_bytes(t.type, t.width) * t.rows));
    qko_synth_superblocks(bytes.data(), t.type, t.rows, t.width, seed,
                          t.type == GGML_TYPE_Q4_K ? 0.01f : 0.005f, 0.01f);
    return bytes;
}

// src/tests/reference/MatmulReference.hpp:31-39
std::vector<float> make_input(size_t count) {
    std::vector<float> input(count);
    for (size_t i = 0; i < count; ++i) input[i] = std::sin(float(i) * 0.031f) * 0.1f;
    return input;
}

std::vector<double> reference(const std::vector<float>& x, const std::vector<unsigned char>& w,
                              const Tensor& t, int64_t rows, int64_t columns) {
    std::vector<double> y(static_cast<size_t>(rows * columns));
    REQUIRE(qko_reference_product(x.data(), w.data(), t.type, t.width, columns, rows, y.data(), 0) == 0);
    return y;
}

void copy_to_host(const DeviceBuffer& source, std::vector<float>& destination) {
    REQUIRE(qk_memcpy_d2h(destination.data(), source.data, destination.size() * sizeof(float), nullptr) == QK_OK);
}

// Catch2 Approx(e).margin(m).epsilon(1e-4) (MatmulReference.hpp:71-79)
void require_product(const std::vector<float>& actual, const std::vector<double>& expected,
                     size_t offset = 0, double margin = 3e-5) {
    REQUIRE(actual.size() >= offset + expected.size());
    for (size_t i = 0; i < expected.size(); ++i) {
        const double diff = std::fabs(double(actual[offset + i]) - expected[i]);
        if (!(diff <= margin || diff <= 1e-4 * std::fabs(expected[i]))) {
            std::printf("  index %zu: actual %.9g expected %.9g\n", i, actual[offset + i], expected[i]);
            REQUIRE(false);
        }
    }
}

}  // namespace

TEST_CASE("Matmul Q4_K and Q6_K match the CPU reference and overwrite reused output") {
    uint64_t seed = 20261201;
    for (const auto& t : kTensors) {
        std::printf("  %s\n", t.name);
        const auto bytes = synth(t, seed++);
        Weight weight(t.name, t.type, {t.width, t.rows}, bytes.data(), bytes.size());
        const size_t width = weight.dimension[0];
        constexpr size_t columns = 5;
        constexpr size_t rows = 3;
        weight.dimension[1] = columns;
        const auto input = make_input(rows * width);
        const auto expected = reference(input, bytes, t, rows, columns);

        DeviceBuffer device_input(input.data(), input.size() * sizeof(float));
        std::vector<float> actual(rows * columns, 123.0f);
        DeviceBuffer device_output(actual.data(), actual.size() * sizeof(float));
        for (int repeat = 0; repeat < 2; ++repeat) {
            kernels::matmul(static_cast<const float*>(device_input.data), weight,
                            static_cast<float*>(device_output.data), rows);
            copy_to_host(device_output, actual);
            require_product(actual, expected, 0, 1e-5);
        }

        DeviceBuffer other_output(actual.data(), actual.size() * sizeof(float));
        kernels::CudaStream first, second;
        kernels::matmul(static_cast<const float*>(device_input.data), weight,
                        static_cast<float*>(device_output.data), rows, first);
        kernels::matmul(static_cast<const float*>(device_input.data), weight,
                        static_cast<float*>(other_output.data), rows, second);
        first.synchronize();
        second.synchronize();
        for (const auto* buffer : {&device_output, &other_output}) {
            copy_to_host(*buffer, actual);
            require_product(actual, expected, 0, 1e-5);
        }

        REQUIRE(qk_memset_async(device_input.data, 0, input.size() * sizeof(float), nullptr) == QK_OK);
        kernels::matmul(static_cast<const float*>(device_input.data), weight,
                        static_cast<float*>(device_output.data), 1);
        std::vector<float> head(columns);
        REQUIRE(qk_memcpy_d2h(head.data(), device_output.data, columns * sizeof(float), nullptr) == QK_OK);
        for (float v : head) REQUIRE(v == 0.0f);
    }
}

TEST_CASE("Matmul matches the quantized CPU reference across row counts") {
    uint64_t seed = 20261301;
    for (const auto& t : kTensors) {
        for (size_t rows : {size_t{1}, size_t{4}, size_t{5}, size_t{101}}) {
            std::printf("  %s rows=%zu\n", t.name, rows);
            const auto bytes = synth(t, seed++);
            Weight weight(t.name, t.type, {t.width, t.rows}, bytes.data(), bytes.size());
            const size_t width = weight.dimension[0];
            constexpr size_t columns = 19;
            weight.dimension[1] = columns;
            const auto input = make_input(rows * width);
            const auto expected = reference(input, bytes, t, rows, columns);
            DeviceBuffer device_input(input.data(), input.size() * sizeof(float));
            std::vector<float> actual(rows * columns + 2, 123.0f);
            DeviceBuffer output(actual.data(), actual.size() * sizeof(float));
            float* product = static_cast<float*>(output.data) + 1;
            kernels::CudaStream stream;
            for (int repeat = 0; repeat < 2; ++repeat) {
                kernels::matmul(static_cast<const float*>(device_input.data), weight, product, rows, stream);
                stream.synchronize();
                copy_to_host(output, actual);
                REQUIRE(actual.front() == 123.0f);
                REQUIRE(actual.back() == 123.0f);
                require_product(actual, expected, 1);
            }
            REQUIRE(qk_memset_async(device_input.data, 0, input.size() * sizeof(float), nullptr) == QK_OK);
            kernels::matmul(static_cast<const float*>(device_input.data), weight, product, rows);
            copy_to_host(output, actual);
            for (size_t i = 0; i < expected.size(); ++i) REQUIRE(actual[i + 1] == 0.0f);
        }
    }
}

TEST_CASE("argmax returns the first index of the largest logit and ignores NaN") {
    std::vector<float> logits(200000);
    for (size_t i = 0; i < logits.size(); ++i) logits[i] = static_cast<float>((i * 7919) % 1000) * 0.5f;
    logits[123457] = 1e6f;
    logits[170001] = 1e6f;  // tie: the lower index wins
    logits[9] = std::numeric_limits<float>::quiet_NaN();
    DeviceBuffer d(logits.size() * sizeof(float));
    kernels::detail::check_status(qk_memcpy_h2d(d.data, logits.data(), logits.size() * sizeof(float), nullptr), "copy");
    REQUIRE(kernels::argmax(static_cast<const float*>(d.data), logits.size()) == 123457u);
    std::vector<float> nothing(33, -std::numeric_limits<float>::infinity());
    nothing[4] = std::numeric_limits<float>::quiet_NaN();
    kernels::detail::check_status(qk_memcpy_h2d(d.data, nothing.data(), nothing.size() * sizeof(float), nullptr), "copy");
    REQUIRE(kernels::argmax(static_cast<const float*>(d.data), nothing.size()) == 0xFFFFFFFFu);
}

TEST_CASE("Streams report readiness and moved-from streams throw") {
    kernels::Stream a;
    a.synchronize();
    REQUIRE(a.ready());
    kernels::Stream b(std::move(a));
    REQUIRE_THROWS_AS(a.get(), std::logic_error);
    REQUIRE(b.get() != nullptr);
    REQUIRE(kernels::detail::get_sm_count() > 0);
}

TEST_CASE("Weights load from a GGUF file and dequantize bit-exactly") {
    const Tensor t{"blk.3.ffn_gate.weight", GGML_TYPE_Q4_K, 2560, 40};
    const auto bytes = synth(t, 77);
    // minimal GGUF v3: one tensor, default alignment 32
    std::vector<unsigned char> file;
    auto pod = [&](auto v) {
        const auto* p = reinterpret_cast<const unsigned char*>(&v);
        file.insert(file.end(), p, p + sizeof(v));
    };
    auto str = [&](const std::string& s) {
        pod(uint64_t(s.size()));
        file.insert(file.end(), s.begin(), s.end());
    };
    file.insert(file.end(), {'G', 'G', 'U', 'F'});
    pod(uint32_t(3)); pod(uint64_t(1)); pod(uint64_t(0));
    str(t.name); pod(uint32_t(2)); pod(int64_t(t.width)); pod(int64_t(t.rows));
    pod(uint32_t(t.type)); pod(uint64_t(0));
    while (file.size() % 32) file.push_back(0);
    file.insert(file.end(), bytes.begin(), bytes.end());
    const auto path = std::filesystem::temp_directory_path() / "qk_matmul_test.gguf";
    {
        std::ofstream f(path, std::ios::binary);
        f.write(reinterpret_cast<const char*>(file.data()), static_cast<std::streamsize>(file.size()));
    }
    const GGUF model(path);
    const Weight weight(model, t.name);
    REQUIRE(weight.datatype == GGML_TYPE_Q4_K && weight.dimension[0] == 2560 && weight.dimension[1] == 40);
    std::vector<float> expected(static_cast<size_t>(t.rows * t.width));
    REQUIRE(qko_dequantize_rows(bytes.data(), expected.data(), t.rows, t.width, 1440, t.type) == 0);
    DeviceBuffer out(expected.size() * sizeof(float));
    kernels::dequantize_embeddings(weight.device_buffer.data, static_cast<float*>(out.data), t.rows,
                                   t.width, 1440, t.type);
    std::vector<float> actual(expected.size());
    copy_to_host(out, actual);
    REQUIRE(std::memcmp(actual.data(), expected.data(), actual.size() * sizeof(float)) == 0);
    std::filesystem::remove(path);
}

namespace {

// A GGUF v3 file with one 2-D tensor (default alignment 32).
std::filesystem::path write_gguf(const char* file_name, const std::string& tensor, ggml_type type,
                                 int64_t width, int64_t rows, const std::vector<unsigned char>& bytes) {
    std::vector<unsigned char> file;
    auto pod = [&](auto v) {
        const auto* p = reinterpret_cast<const unsigned char*>(&v);
        file.insert(file.end(), p, p + sizeof(v));
    };
    auto str = [&](const std::string& s) {
        pod(uint64_t(s.size()));
        file.insert(file.end(), s.begin(), s.end());
    };
    file.insert(file.end(), {'G', 'G', 'U', 'F'});
    pod(uint32_t(3)); pod(uint64_t(1)); pod(uint64_t(0));
    str(tensor); pod(uint32_t(2)); pod(int64_t(width)); pod(int64_t(rows));
    pod(uint32_t(type)); pod(uint64_t(0));
    while (file.size() % 32) file.push_back(0);
    file.insert(file.end(), bytes.begin(), bytes.end());
    const auto path = std::filesystem::temp_directory_path() / file_name;
    std::ofstream f(path, std::ios::binary);
    f.write(reinterpret_cast<const char*>(file.data()), static_cast<std::streamsize>(file.size()));
    return path;
}

}  // namespace

TEST_CASE("EmbedLookup gathers rows in input order and dequantizes them bit-exactly") {
    // src/tests/EmbedLookupTests.cpp:10-52 on a synthetic token_embd of each storage type
    for (const ggml_type type : {GGML_TYPE_Q6_K, GGML_TYPE_Q4_K, GGML_TYPE_F32}) {
        const int64_t width = 2560, vocabulary = 64;
        const int64_t row_bytes = ggml_row_bytes(type, width);
        std::vector<unsigned char> table(static_cast<size_t>(row_bytes * vocabulary));
        if (type == GGML_TYPE_F32) {
            for (size_t i = 0; i < table.size() / 4; ++i) {
                const float v = std::sin(float(i) * 0.37f);
                std::memcpy(table.data() + 4 * i, &v, 4);
            }
        } else {
            qko_synth_superblocks(table.data(), type, vocabulary, width, 4242 + type,
                                  type == GGML_TYPE_Q4_K ? 0.01f : 0.005f, 0.01f);
        }
        const auto path = write_gguf("qk_embed_test.gguf", "token_embd.weight", type, width, vocabulary, table);
        const GGUF model(path);
        const EmbedLookup lookup(model);
        REQUIRE(lookup.get_embedding_size() == size_t(width));
        REQUIRE(lookup.get_vocabulary_size() == size_t(vocabulary));
        REQUIRE(lookup.get_row_bytes() == size_t(row_bytes));
        const auto empty = lookup.lookup({});
        REQUIRE(empty.bytes == 0 && empty.data == nullptr);
        REQUIRE_THROWS_AS(lookup.lookup({std::numeric_limits<uint32_t>::max()}), std::out_of_range);
        REQUIRE_THROWS_AS(lookup.lookup({3, 64}), std::out_of_range);
        std::vector<uint32_t> ids;  // repeated ids, out of order
        for (uint32_t i = 0; i < 32; ++i) ids.push_back(i % 3 == 0 ? 42 : i % 3 == 1 ? 7 : 63 - i);
        const auto device = lookup.lookup(ids);
        REQUIRE(device.bytes == ids.size() * width * sizeof(float));
        std::vector<float> actual(ids.size() * width), expected(width);
        REQUIRE(qk_memcpy_d2h(actual.data(), device.data, device.bytes, nullptr) == QK_OK);
        for (size_t r = 0; r < ids.size(); ++r) {
            const unsigned char* row = table.data() + ids[r] * row_bytes;
            if (type == GGML_TYPE_F32) std::memcpy(expected.data(), row, width * 4);
            else REQUIRE(qko_dequantize_rows(row, expected.data(), 1, width, row_bytes, type) == 0);
            REQUIRE(std::memcmp(actual.data() + r * width, expected.data(), width * sizeof(float)) == 0);
        }
        std::filesystem::remove(path);
    }
}

TEST_CASE("rms_norm and residual_add match the CPU oracle") {
    // src/cuda/rms_norm.cu:6-36 and src/cuda/residual_add.cu:6-20
    const size_t rows = 5, width = 2560;
    const float eps = 1e-6f;
    std::vector<float> x(rows * width), scale(width), branch(rows * width);
    for (size_t i = 0; i < x.size(); ++i) {
        x[i] = std::sin(float(i) * 0.031f) * (1.0f + float(i % 7));
        branch[i] = std::cos(float(i) * 0.017f);
    }
    for (size_t i = 0; i < width; ++i) scale[i] = 1.0f + 0.5f * std::sin(float(i));
    const Weight norm("blk.0.ffn_norm.weight", GGML_TYPE_F32, {int64_t(width)}, scale.data(), width * 4);
    DeviceBuffer xd(x.data(), x.size() * 4), out(x.size() * 4), bd(branch.data(), branch.size() * 4);
    kernels::rms_norm(static_cast<float*>(xd.data), norm, static_cast<float*>(out.data), rows, width, eps);
    std::vector<float> got(x.size()), expected(x.size());
    copy_to_host(out, got);
    qko_rms_norm(x.data(), scale.data(), expected.data(), rows, width, eps);
    for (size_t i = 0; i < got.size(); ++i)
        REQUIRE(std::fabs(got[i] - expected[i]) <= 2e-6f * std::fabs(expected[i]) + 1e-30f);
    REQUIRE_THROWS_AS(kernels::rms_norm(static_cast<float*>(xd.data), norm, static_cast<float*>(out.data),
                                        rows, width + 256, eps),
                      std::invalid_argument);  // scale width mismatch
    REQUIRE_THROWS_AS(kernels::rms_norm(static_cast<float*>(xd.data), norm, static_cast<float*>(out.data),
                                        rows, width, 0.0f),
                      std::invalid_argument);
    kernels::residual_add(static_cast<float*>(xd.data), static_cast<float*>(bd.data), x.size());
    copy_to_host(xd, got);
    for (size_t i = 0; i < got.size(); ++i) REQUIRE(got[i] == x[i] + branch[i]);
    kernels::detail::check_launch();
}

int main() { return mini::run_all(); }
