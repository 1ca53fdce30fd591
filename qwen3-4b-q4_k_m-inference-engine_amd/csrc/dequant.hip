// Superblock rows -> fp32, bit-identical to the per-element formulas of
// src/cuda/embedding.cu:6-59 (Q4_K: (d*sc)*q - dmin*m; Q6_K: (d*sc)*(q-32)).
// Every product there is exact in fp32 (an fp16 d times a <= 6-bit scale
// times a <= 6-bit code), so contraction into fma cannot change a bit.
// One wave per superblock; lane l writes weights 4l..4l+3 as one float4.
#include "qk_device.hpp"
#include "qk_launch.hpp"

namespace qk {
namespace {

__device__ __forceinline__ uint32_t load_bytes4(const uint8_t* p) {
  return static_cast<uint32_t>(p[0]) | (static_cast<uint32_t>(p[1]) << 8) |
         (static_cast<uint32_t>(p[2]) << 16) | (static_cast<uint32_t>(p[3]) << 24);
}

__device__ __forceinline__ f32x4 dequant4_q4k(const uint8_t* block, uint32_t l) {
  const uint32_t g = l >> 3;            // sub-block of weights 4l..4l+3
  const uint32_t pos = 4u * (l & 7u);   // position inside the sub-block
  const uint32_t qs = load_bytes4(block + 16 + (g >> 1) * 32 + pos);
  const uint32_t s0 = load_bytes4(block + 4);
  const uint32_t s1 = load_bytes4(block + 8);
  const uint32_t s2 = load_bytes4(block + 12);
  int sc, m;
  scale_min_k4(g, s0, s1, s2, sc, m);
  const float d = half_bits_to_float(load_bytes4(block) & 0xFFFFu);
  const float dmin = half_bits_to_float(load_bytes4(block) >> 16);
  const float ds = d * static_cast<float>(sc);
  const float dm = dmin * static_cast<float>(m);
  const uint32_t q = (qs >> ((g & 1u) * 4u)) & 0x0F0F0F0Fu;
  f32x4 out;
  out.x = ds * static_cast<float>(q & 0xFFu) - dm;
  out.y = ds * static_cast<float>((q >> 8) & 0xFFu) - dm;
  out.z = ds * static_cast<float>((q >> 16) & 0xFFu) - dm;
  out.w = ds * static_cast<float>(q >> 24) - dm;
  return out;
}

__device__ __forceinline__ f32x4 dequant4_q6k(const uint8_t* block, uint32_t l) {
  const uint32_t half = l >> 5;          // weights 4l..4l+3: p/128
  const uint32_t group = (l & 31u) >> 3; // (p%128)/32
  const uint32_t pos = 4u * (l & 7u);    // p%32
  const uint32_t low =
      (load_bytes4(block + half * 64 + (group & 1u) * 32 + pos) >> (4u * (group >> 1))) &
      0x0F0F0F0Fu;
  const uint32_t high = (load_bytes4(block + 128 + half * 32 + pos) >> (2u * group)) & 0x03030303u;
  const uint32_t codes = low | (high << 4);
  const int scale = static_cast<int8_t>(block[192 + (l >> 2)]);  // p/16
  const float d = half_bits_to_float(static_cast<uint32_t>(block[208]) |
                                     (static_cast<uint32_t>(block[209]) << 8));
  const float ds = d * static_cast<float>(scale);
  f32x4 out;
  out.x = ds * static_cast<float>(static_cast<int>(codes & 0xFFu) - 32);
  out.y = ds * static_cast<float>(static_cast<int>((codes >> 8) & 0xFFu) - 32);
  out.z = ds * static_cast<float>(static_cast<int>((codes >> 16) & 0xFFu) - 32);
  out.w = ds * static_cast<float>(static_cast<int>(codes >> 24) - 32);
  return out;
}

template <int TYPE>
__global__ __launch_bounds__(256) void dequantize_kernel(const uint8_t* __restrict__ packed,
                                                         float* __restrict__ out,
                                                         int64_t total_blocks, int64_t sb_per_row,
                                                         int64_t row_bytes) {
  constexpr int kBytes = TYPE == QK_TYPE_Q4_K ? kQ4KBytes : kQ6KBytes;
  const uint32_t l = threadIdx.x & 63u;
  const int64_t waves = static_cast<int64_t>(gridDim.x) * 4;
  for (int64_t b = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6); b < total_blocks;
       b += waves) {
    const int64_t row = b / sb_per_row;
    const int64_t s = b - row * sb_per_row;
    const uint8_t* block = packed + row * row_bytes + s * kBytes;
    const f32x4 v = TYPE == QK_TYPE_Q4_K ? dequant4_q4k(block, l) : dequant4_q6k(block, l);
    // out is only required to be 4-byte aligned, like any float*
    *reinterpret_cast<f32x4_a4*>(out + b * kQK + 4 * l) = v;
  }
}

}  // namespace

hipError_t launch_dequantize_rows(const void* packed, float* out, int64_t rows, int64_t K,
                                  size_t row_bytes, int type, hipStream_t stream) {
  const int64_t sb = K / kQK;
  const int64_t total = rows * sb;
  const int64_t grid = total / 4 + 1 < 65536 ? total / 4 + 1 : 65536;
  const auto* bytes = static_cast<const uint8_t*>(packed);
  if (type == QK_TYPE_Q4_K)
    dequantize_kernel<QK_TYPE_Q4_K><<<dim3(static_cast<uint32_t>(grid)), dim3(256), 0, stream>>>(
        bytes, out, total, sb, static_cast<int64_t>(row_bytes));
  else
    dequantize_kernel<QK_TYPE_Q6_K><<<dim3(static_cast<uint32_t>(grid)), dim3(256), 0, stream>>>(
        bytes, out, total, sb, static_cast<int64_t>(row_bytes));
  return hipGetLastError();
}

}  // namespace qk
