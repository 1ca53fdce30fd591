// Compile-and-link check of the drop-in headers: the reference engine's
// per-token call sequence (src/Engine.cpp:55-111: embedding lookup, per layer
// rms_norm, q/k/v matmuls, q/k norms, rope, attention, attn_output, residual,
// ffn_norm, gate/up, silu_multiply, down, residual; then output_norm, lm_head
// and argmax) written against include/ only, with the reference's argument
// kinds. It is built and linked against libqk_engine.so, never run: rope and
// attention stay with the engine, so this file gives them empty bodies, and the
// KV cache below stands in for the engine's ChatSession (include/ChatSession.hpp).
#include <cstdint>
#include <string>
#include <unordered_map>
#include <vector>

#include "EmbedLookup.hpp"
#include "GGUF.hpp"
#include "Kernels.hpp"
#include "Weight.hpp"

namespace kernels {
void rope(float*, size_t, size_t, size_t, size_t, float) {}
void attention(const float*, const float*, const float*, float*, size_t, size_t, size_t, size_t,
               size_t) {}
}  // namespace kernels

namespace {

struct KvCache {
    std::unordered_map<std::string, DeviceBuffer> slots;
    size_t cached = 0;
    float* base(const std::string& name) { return static_cast<float*>(slots.at(name).data); }
};

uint32_t decode(const GGUF& gguf, const std::unordered_map<std::string, Weight>& weights,
                const EmbedLookup& embed, KvCache& cache, const std::vector<uint32_t>& pending) {
    using namespace kernels;
    const size_t tokens = pending.size();
    const size_t offset = cache.cached;
    const size_t width = embed.get_embedding_size();
    const size_t heads = gguf.get_attention_head_count().value();
    const size_t kv_heads = gguf.get_value<uint32_t>("qwen3.attention.head_count_kv").value();
    const size_t head_dim = gguf.get_value<uint32_t>("qwen3.attention.key_length").value();
    const size_t ffn_width = gguf.get_value<uint32_t>("qwen3.feed_forward_length").value();
    const float epsilon = gguf.get_value<float>("qwen3.attention.layer_norm_rms_epsilon").value();
    const float rope_base = gguf.get_value<float>("qwen3.rope.freq_base").value();

    DeviceBuffer state{embed.lookup(pending)};
    auto buffer = [](size_t floats) { return DeviceBuffer(floats * sizeof(float)); };
    DeviceBuffer normalized = buffer(tokens * width), q = buffer(tokens * heads * head_dim);
    DeviceBuffer k = buffer(tokens * kv_heads * head_dim), qn = buffer(tokens * heads * head_dim);
    DeviceBuffer attended = buffer(tokens * heads * head_dim), branch = buffer(tokens * width);
    DeviceBuffer gate = buffer(tokens * ffn_width), up = buffer(tokens * ffn_width);
    DeviceBuffer activated = buffer(tokens * ffn_width);
    auto f = [](DeviceBuffer& b) { return static_cast<float*>(b.data); };

    for (size_t layer = 0; layer < gguf.get_layer_count().value(); ++layer) {
        auto w = [&](const char* name) -> const Weight& {
            return weights.at("blk." + std::to_string(layer) + "." + name);
        };
        const std::string key = "blk." + std::to_string(layer) + ".key";
        const std::string value = "blk." + std::to_string(layer) + ".value";
        float* cached_k = cache.base(key);
        float* cached_v = cache.base(value);
        float* new_k = cached_k + offset * kv_heads * head_dim;
        float* new_v = cached_v + offset * kv_heads * head_dim;

        rms_norm(f(state), w("attn_norm.weight"), f(normalized), tokens, width, epsilon);
        matmul(f(normalized), w("attn_q.weight"), f(q), tokens);
        matmul(f(normalized), w("attn_k.weight"), f(k), tokens);
        matmul(f(normalized), w("attn_v.weight"), new_v, tokens);
        rms_norm(f(q), w("attn_q_norm.weight"), f(qn), tokens * heads, head_dim, epsilon);
        rms_norm(f(k), w("attn_k_norm.weight"), new_k, tokens * kv_heads, head_dim, epsilon);
        rope(f(qn), tokens, heads, head_dim, offset, rope_base);
        rope(new_k, tokens, kv_heads, head_dim, offset, rope_base);
        attention(f(qn), cached_k, cached_v, f(attended), tokens, heads, kv_heads, head_dim, offset);
        matmul(f(attended), w("attn_output.weight"), f(branch), tokens);
        residual_add(f(state), f(branch), tokens * width);
        rms_norm(f(state), w("ffn_norm.weight"), f(normalized), tokens, width, epsilon);
        matmul(f(normalized), w("ffn_gate.weight"), f(gate), tokens);
        matmul(f(normalized), w("ffn_up.weight"), f(up), tokens);
        silu_multiply(f(gate), f(up), f(activated), tokens * ffn_width);
        matmul(f(activated), w("ffn_down.weight"), f(branch), tokens);
        residual_add(f(state), f(branch), tokens * width);
    }
    rms_norm(f(state) + (tokens - 1) * width, weights.at("output_norm.weight"), f(normalized), 1,
             width, epsilon);
    DeviceBuffer logits = buffer(embed.get_vocabulary_size());
    matmul(f(normalized), weights.at("token_embd.weight"), f(logits), 1);
    detail::check_launch();
    cache.cached += tokens;
    return argmax(f(logits), embed.get_vocabulary_size());
}

}  // namespace

int main(int argc, char** argv) {
    if (argc < 2) return 0;
    const GGUF gguf(argv[1], false);
    std::unordered_map<std::string, Weight> weights;
    for (const auto& tensor : gguf.get_tensors()) weights.try_emplace(tensor.name, gguf, tensor.name);
    const EmbedLookup embed(gguf);
    KvCache cache;
    kernels::CudaStream stream;
    stream.synchronize();
    return static_cast<int>(decode(gguf, weights, embed, cache, {1, 2, 3}) == 0xFFFFFFFFu);
}
