// Device-side building blocks for the gfx950 Q4_K/Q6_K kernels: superblock
// layouts, vector loads, the 6-bit scale unpack, fp16 widening and wave64
// DPP reductions. Written for CDNA4 (wave64, v_dot4_i32_i8, DPP row ops).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "qk_abi.h"

namespace qk {

constexpr int kQK = 256;        // weights per superblock
constexpr int kQ4KBytes = 144;  // d, dmin, scales[12], qs[128]
constexpr int kQ6KBytes = 210;  // ql[128], qh[64], scales[16], d

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
// The same vectors at 2-byte alignment: Q6_K superblocks sit at 210*s, so odd
// superblocks of a row start 2 bytes off a dword boundary. gfx950 global
// loads accept unaligned addresses; the compiler emits one dwordx4 for these.
typedef u32x4 u32x4_a2 __attribute__((aligned(2)));
typedef u32x4 u32x4_a4 __attribute__((aligned(4)));
typedef f32x4 f32x4_a4 __attribute__((aligned(4)));

static_assert(sizeof(qk_q8_block) == 48, "Q8 block is 48 bytes");

__device__ __forceinline__ u32x4 load16(const void* p) {
  return *reinterpret_cast<const u32x4*>(p);
}
__device__ __forceinline__ u32x4 load16_a2(const void* p) {
  return *reinterpret_cast<const u32x4_a2*>(p);
}
__device__ __forceinline__ uint32_t load_u16(const void* p) {
  return *reinterpret_cast<const uint16_t*>(p);
}
__device__ __forceinline__ u32x4 load16_a4(const void* p) {
  return *reinterpret_cast<const u32x4_a4*>(p);
}
__device__ __forceinline__ uint32_t load_u32(const void* p) {
  return *reinterpret_cast<const uint32_t*>(p);
}

// fp16 bits -> fp32 (exact, subnormals kept: the kernels run with fp16
// denormals enabled, which is the gfx950 default mode).
__device__ __forceinline__ float half_bits_to_float(uint32_t bits) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits)));
}

__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int acc) {
  return __builtin_amdgcn_sdot4(static_cast<int>(a), static_cast<int>(b), acc, false);
}

__device__ __forceinline__ uint32_t ubfe(uint32_t v, uint32_t offset, uint32_t width) {
  return __builtin_amdgcn_ubfe(v, offset, width);
}

// 6-bit (scale, min) of Q4_K sub-block g from the 12-byte field held in the
// three header dwords s0 = scales[0..3], s1 = scales[4..7], s2 = scales[8..11].
// Same bits as get_scale_min_k4 (src/cuda/embedding.cu:20-23):
//   g < 4 : sc = scales[g] & 63,            m = scales[g+4] & 63
//   g >= 4: sc = (scales[g+4] & 15) | (scales[g-4] >> 6) << 4
//           m  = (scales[g+4] >> 4) | (scales[g]   >> 6) << 4
// Branch-free: a zero-width bit-field extract yields 0, which drops the high
// part for g < 4.
__device__ __forceinline__ void scale_min_k4(uint32_t g, uint32_t s0, uint32_t s1, uint32_t s2,
                                             int& sc, int& m) {
  const uint32_t hi = g >> 2;
  const uint32_t pos = (g & 3u) * 8u;
  const uint32_t low_width = hi ? 4u : 6u;
  const uint32_t high_width = hi ? 2u : 0u;
  const uint32_t sc_src = hi ? s2 : s0;
  const uint32_t m_src = hi ? s2 : s1;
  const uint32_t m_pos = pos + (hi ? 4u : 0u);
  sc = static_cast<int>(ubfe(sc_src, pos, low_width) | (ubfe(s0, pos + 6u, high_width) << 4));
  m = static_cast<int>(ubfe(m_src, m_pos, low_width) | (ubfe(s1, pos + 6u, high_width) << 4));
}

// Sum over the 8 lanes of each aligned lane octet (quad swaps, then the
// half-row mirror); every lane of the octet receives the sum.
__device__ __forceinline__ float octet_sum(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                             0xB1, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                             0x4E, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                             0x141, 0xF, 0xF, false));
  return v;
}

// Register images of what one lane reads per superblock. Loads and math are
// split so a wave can issue every load of several superblocks before it
// consumes the first one.
struct XFrag {  // one Q8 activation block
  u32x4 c0, c1, rec;
};
struct Q4KFrag {  // header + the 32 qs bytes holding sub-blocks 2j, 2j+1
  u32x4 head, q0, q1;
};
// Q6_K superblocks sit at 210*s, so odd ones start 2 bytes off a dword.
// 16-byte loads at 2-byte alignment run far slower than dword-aligned ones,
// so every Q6_K load starts on the dword boundary at or below its field
// (36 bytes cover 32 field bytes) and v_alignbit realigns in registers.
struct Q6KFrag {  // 32 ql bytes, 32 qh bytes, the two int8 scales, d
  u32x4 l0, l1, h0, h1;
  uint32_t l2, h2;   // the dwords after l1 / h1
  uint32_t sc_word;  // dword holding scales[8h+2g], scales[8h+2g+1]
  uint32_t d_bits;   // d (2-byte load: a dword could pass the superblock's end)
  uint32_t shift;    // field misalignment in bits: 0 or 16
  uint32_t sc_shift; // bit offset of the scale pair in sc_word: 0 or 16
};

__device__ __forceinline__ XFrag load_x(const qk_q8_block* __restrict__ xb) {
  XFrag f;
  f.c0 = load16(xb->codes);
  f.c1 = load16(xb->codes + 16);
  f.rec = load16(&xb->scale);
  return f;
}

__device__ __forceinline__ Q4KFrag load_q4k(const uint8_t* __restrict__ sb, uint32_t g) {
  Q4KFrag f;
  f.head = load16(sb);                              // d, dmin, scales[0..11]
  const uint8_t* qs = sb + 16 + 32 * (g >> 1);
  f.q0 = load16(qs);
  f.q1 = load16(qs + 16);
  return f;
}

// Q6_K lane c covers Q8 block c: h = c/4 selects the 128-weight half, g = c%4
// the 32-weight group, i.e. the two 16-weight scale groups 8h+2g, 8h+2g+1.
__device__ __forceinline__ Q6KFrag load_q6k(const uint8_t* __restrict__ sb, uint32_t c) {
  const uint32_t h = c >> 2;
  const uint32_t g = c & 3u;
  const uint32_t mis = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(sb)) & 3u;  // 0 or 2
  const uint8_t* base = sb - mis;  // dword-aligned
  const uint8_t* ql = base + 64 * h + 32 * (g & 1u);
  const uint8_t* qh = base + 128 + 32 * h;
  Q6KFrag f;
  f.l0 = load16_a4(ql);
  f.l1 = load16_a4(ql + 16);
  f.l2 = load_u32(ql + 32);
  f.h0 = load16_a4(qh);
  f.h1 = load16_a4(qh + 16);
  f.h2 = load_u32(qh + 32);
  // The scale pair's dword spans at most bytes 204..209 of the superblock.
  // Shifts are applied in dot_q6k: using a loaded value here would make the
  // wave wait for the load before it can issue the next superblock's loads.
  const uint32_t sc_off = 192 + 8 * h + 2 * g + mis;  // from base
  f.sc_word = load_u32(base + (sc_off & ~3u));
  f.sc_shift = 8 * (sc_off & 3u);
  f.d_bits = load_u16(sb + 208);
  f.shift = 8 * mis;
  return f;
}

// Sub-block g (32 weights) of a Q4_K superblock against its Q8 block:
// xs*(d*sc*dot) - dmin*m*(xs*sum(codes)), the sub-block's term of the
// reference's per-superblock sum (src/cuda/matmul.cu:24-54).
__device__ __forceinline__ float dot_q4k(const Q4KFrag& w, const XFrag& x, uint32_t g) {
  const uint32_t shift = (g & 1u) * 4u;  // low nibble: even g, high: odd g
  constexpr uint32_t kNib = 0x0F0F0F0Fu;
  int dot = dot4((w.q0.x >> shift) & kNib, x.c0.x, 0);
  dot = dot4((w.q0.y >> shift) & kNib, x.c0.y, dot);
  dot = dot4((w.q0.z >> shift) & kNib, x.c0.z, dot);
  dot = dot4((w.q0.w >> shift) & kNib, x.c0.w, dot);
  dot = dot4((w.q1.x >> shift) & kNib, x.c1.x, dot);
  dot = dot4((w.q1.y >> shift) & kNib, x.c1.y, dot);
  dot = dot4((w.q1.z >> shift) & kNib, x.c1.z, dot);
  dot = dot4((w.q1.w >> shift) & kNib, x.c1.w, dot);
  int sc, m;
  scale_min_k4(g, w.head.y, w.head.z, w.head.w, sc, m);
  const float d = half_bits_to_float(w.head.x & 0xFFFFu);
  const float dmin = half_bits_to_float(w.head.x >> 16);
  const f32x4 rec = __builtin_bit_cast(f32x4, x.rec);
  // |sc*dot| <= 63*32*15*127 < 2^24, so the integer product converts exactly.
  const float main_term = d * static_cast<float>(__mul24(sc, dot));
  return main_term * rec.x - (dmin * static_cast<float>(m)) * rec.y;
}

// Q8 block c of a Q6_K superblock (src/cuda/matmul.cu:61-84):
//   q = ((ql >> 4*(g/2)) & 15) | ((qh >> 2g) & 3) << 4, weight = d*sc*(q-32).
// The -32 offset enters through the Q8 block's neg32 sums as the dots' start.
__device__ __forceinline__ float dot_q6k(const Q6KFrag& w, const XFrag& x, uint32_t c) {
  const uint32_t g = c & 3u;
  const i32x4 rec = __builtin_bit_cast(i32x4, x.rec);
  const uint32_t sh = w.shift;
  auto realign = [sh](uint32_t hi, uint32_t lo) { return __builtin_amdgcn_alignbit(hi, lo, sh); };
  const uint32_t l[8] = {realign(w.l0.y, w.l0.x), realign(w.l0.z, w.l0.y), realign(w.l0.w, w.l0.z),
                         realign(w.l1.x, w.l0.w), realign(w.l1.y, w.l1.x), realign(w.l1.z, w.l1.y),
                         realign(w.l1.w, w.l1.z), realign(w.l2, w.l1.w)};
  const uint32_t q[8] = {realign(w.h0.y, w.h0.x), realign(w.h0.z, w.h0.y), realign(w.h0.w, w.h0.z),
                         realign(w.h1.x, w.h0.w), realign(w.h1.y, w.h1.x), realign(w.h1.z, w.h1.y),
                         realign(w.h1.w, w.h1.z), realign(w.h2, w.h1.w)};
  const uint32_t lo_shift = 4u * (g >> 1);
  // rotate so bits (2g, 2g+1) of every byte land on bits 4 and 5
  const uint32_t hi_rot = (2u * g - 4u) & 31u;
  constexpr uint32_t kLo = 0x0F0F0F0Fu, kHi = 0x30303030u;
  auto code = [&](uint32_t l, uint32_t h) {
    return ((l >> lo_shift) & kLo) | (__builtin_amdgcn_alignbit(h, h, hi_rot) & kHi);
  };
  int dot_lo = dot4(code(l[0], q[0]), x.c0.x, rec.z);
  dot_lo = dot4(code(l[1], q[1]), x.c0.y, dot_lo);
  dot_lo = dot4(code(l[2], q[2]), x.c0.z, dot_lo);
  dot_lo = dot4(code(l[3], q[3]), x.c0.w, dot_lo);
  int dot_hi = dot4(code(l[4], q[4]), x.c1.x, rec.w);
  dot_hi = dot4(code(l[5], q[5]), x.c1.y, dot_hi);
  dot_hi = dot4(code(l[6], q[6]), x.c1.z, dot_hi);
  dot_hi = dot4(code(l[7], q[7]), x.c1.w, dot_hi);
  const uint32_t pair = w.sc_word >> w.sc_shift;
  const int sc0 = static_cast<int>(static_cast<int8_t>(pair & 0xFFu));
  const int sc1 = static_cast<int>(static_cast<int8_t>((pair >> 8) & 0xFFu));
  // |sc*dot| <= 64*16*32*127 per group, the sum < 2^24: exact in fp32.
  const int isum = __mul24(sc0, dot_lo) + __mul24(sc1, dot_hi);
  const float d = half_bits_to_float(w.d_bits);
  return (d * __builtin_bit_cast(float, rec.x)) * static_cast<float>(isum);
}

}  // namespace qk
