// Synthetic superblocks and activations generated in place on the device from
// a counter-based SplitMix64 stream: word(seed, i) = mix64(seed + (i+1)*golden)
// is the i-th output of SplitMix64, so every byte is computed independently.
// Layout of the stream per superblock and per activation: see the
// qk_synth_superblocks declaration in qk_abi.h.
#include "qk_device.hpp"
#include "qk_launch.hpp"

namespace qk {
namespace {

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

__device__ __forceinline__ uint64_t word_at(uint64_t seed, uint64_t i) {
  return mix64(seed + (i + 1) * 0x9E3779B97F4A7C15ull);
}

__device__ __forceinline__ float u24(uint64_t w) {
  return static_cast<float>(w >> 40) * (1.0f / 16777216.0f);
}

// fp16(u24(w) * scale) with the product rounded to fp32 first. The empty asm
// pins the fp32 product in a register: otherwise the compiler fuses the
// multiply into the narrowing (v_fma_mixlo_f16), which rounds once, straight
// to fp16, and breaks fp32-level ties the other way.
__device__ __forceinline__ uint32_t scaled_fp16_bits(uint64_t w, float scale) {
  float product = u24(w) * scale;
  asm volatile("" : "+v"(product));
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(product));
}

__device__ __forceinline__ uint8_t byte_of(uint64_t w, uint32_t i) {
  return static_cast<uint8_t>(w >> (8 * i));
}

// One byte per thread, grid-stride over the tensor.
__global__ __launch_bounds__(256) void synth_q4k_kernel(uint8_t* __restrict__ out, int64_t bytes,
                                                        uint64_t seed, float dmax, float dminmax) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < bytes; i += stride) {
    const int64_t b = i / kQ4KBytes;
    const uint32_t j = static_cast<uint32_t>(i - b * kQ4KBytes);
    const uint64_t base = static_cast<uint64_t>(b) * 20u;
    uint8_t v;
    if (j < 4) {
      const float scale = j < 2 ? dmax : dminmax;
      const uint32_t h = scaled_fp16_bits(word_at(seed, base + (j >> 1)), scale);
      v = static_cast<uint8_t>(h >> (8 * (j & 1u)));
    } else if (j < 16) {
      const uint32_t t = j - 4;
      v = byte_of(word_at(seed, base + 2 + t / 8), t % 8);
    } else {
      const uint32_t t = j - 16;
      v = byte_of(word_at(seed, base + 4 + t / 8), t % 8);
    }
    out[i] = v;
  }
}

__global__ __launch_bounds__(256) void synth_q6k_kernel(uint8_t* __restrict__ out, int64_t bytes,
                                                        uint64_t seed, float dmax) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < bytes; i += stride) {
    const int64_t b = i / kQ6KBytes;
    const uint32_t j = static_cast<uint32_t>(i - b * kQ6KBytes);
    const uint64_t base = static_cast<uint64_t>(b) * 27u;
    uint8_t v;
    if (j < 192) {
      v = byte_of(word_at(seed, base + j / 8), j % 8);
    } else if (j < 208) {
      const uint32_t t = j - 192;
      const int raw = byte_of(word_at(seed, base + 24 + t / 8), t % 8) & 127;
      v = static_cast<uint8_t>(static_cast<int8_t>(raw - 64));
    } else {
      const uint32_t h = scaled_fp16_bits(word_at(seed, base + 26), dmax);
      v = static_cast<uint8_t>(h >> (8 * (j - 208)));
    }
    out[i] = v;
  }
}

__global__ __launch_bounds__(256) void synth_normal_kernel(float* __restrict__ x, int64_t count,
                                                           uint64_t seed) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < count; i += stride) {
    const double u1 = 1.0 - static_cast<double>(u24(word_at(seed, 2 * static_cast<uint64_t>(i))));
    const double u2 = static_cast<double>(u24(word_at(seed, 2 * static_cast<uint64_t>(i) + 1)));
    x[i] = static_cast<float>(sqrt(-2.0 * log(u1)) * cos(6.283185307179586476925286766559 * u2));
  }
}

uint32_t grid_for(int64_t items) {
  const int64_t blocks = (items + 255) / 256;
  return static_cast<uint32_t>(blocks < 16384 ? (blocks > 0 ? blocks : 1) : 16384);
}

}  // namespace

hipError_t launch_synth_superblocks(void* w, int type, int64_t N, int64_t K, uint64_t seed,
                                    float dmax, float dminmax, hipStream_t stream) {
  auto* out = static_cast<uint8_t*>(w);
  const int64_t blocks = N * (K / kQK);
  if (type == QK_TYPE_Q4_K) {
    const int64_t bytes = blocks * kQ4KBytes;
    synth_q4k_kernel<<<grid_for(bytes), 256, 0, stream>>>(out, bytes, seed, dmax, dminmax);
  } else {
    const int64_t bytes = blocks * kQ6KBytes;
    synth_q6k_kernel<<<grid_for(bytes), 256, 0, stream>>>(out, bytes, seed, dmax);
  }
  return hipGetLastError();
}

hipError_t launch_synth_normal(float* x, int64_t count, uint64_t seed, hipStream_t stream) {
  synth_normal_kernel<<<grid_for(count), 256, 0, stream>>>(x, count, seed);
  return hipGetLastError();
}

}  // namespace qk
