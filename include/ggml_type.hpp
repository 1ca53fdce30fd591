#pragma once
// GGUF on-disk tensor type ids. The values are ggml's `enum ggml_type`
// (ggml.h, GIT_TAG master as fetched by the reference's CMakeLists.txt:30-37),
// which the reference reaches through GGUF.hpp:3; they are a file-format
// constant, so the enumerator names and values are kept identical for
// source compatibility with code such as src/Engine.cpp and src/tests/.
#include <cstdint>

enum ggml_type : int32_t {
    GGML_TYPE_F32 = 0,
    GGML_TYPE_F16 = 1,
    GGML_TYPE_Q4_0 = 2,
    GGML_TYPE_Q4_1 = 3,
    GGML_TYPE_Q5_0 = 6,
    GGML_TYPE_Q5_1 = 7,
    GGML_TYPE_Q8_0 = 8,
    GGML_TYPE_Q8_1 = 9,
    GGML_TYPE_Q2_K = 10,
    GGML_TYPE_Q3_K = 11,
    GGML_TYPE_Q4_K = 12,
    GGML_TYPE_Q5_K = 13,
    GGML_TYPE_Q6_K = 14,
    GGML_TYPE_Q8_K = 15,
    GGML_TYPE_BF16 = 30,
    // Past every type id above; code such as src/EmbedLookup.cpp uses it as
    // the "no type" marker.
    GGML_TYPE_COUNT = 40,
};

// Bytes per row of `width` weights for the types this library computes on
// (0 for any other type). Q4_K/Q6_K pack 256 weights per 144/210 bytes.
inline std::int64_t ggml_row_bytes(ggml_type type, std::int64_t width) {
    switch (type) {
    case GGML_TYPE_F32: return width * 4;
    case GGML_TYPE_F16: return width * 2;
    case GGML_TYPE_Q4_K: return width / 256 * 144;
    case GGML_TYPE_Q6_K: return width / 256 * 210;
    default: return 0;
    }
}
