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

// The same loads with the nontemporal hint, for weight bytes that a kernel
// reads exactly once (one instruction per byte): the streamed matrix then does
// not push code, activations and other reused lines out of the caches
// (whole-share mat-vec: 3-5% per decode launch). Not for bytes that several
// instructions read (the streaming mat-vec's pieces share cache lines: there
// the hint made lm_head 2x slower).
__device__ __forceinline__ u32x4 stream_load16_a4(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4_a4*>(p));
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

// Register images of what one lane reads per superblock piece. A piece is a
// quarter of a superblock whose bytes are not shared with the other pieces
// (Q4_K) or share only qh (Q6_K): 64 weights, two Q8 activation blocks.
// Loads and math are split so a wave can issue every load of several pieces
// before it consumes the first one.
struct XFrag {  // one Q8 activation block
  u32x4 c0, c1, rec;
};

// Exact-rounding building blocks of the activation quantiser (Q8 codes and
// scales as the reference computes them in float, for a block maximum amax
// in [2^-64, 2^64]):
//  refined_rcp(a)        = RN(1/a): v_rcp_f32 plus one FMA refinement;
//  markstein_div(x,b,r)  = RN(x/b) given r = RN(1/b) (Markstein's correction);
//  round_code(t)         = roundf(t) for |t| <= 127, as a truncation of
//                          t + copysign(0.49999997f, t);
//  q8_code(x, amax, r)   = roundf(RN(x/amax) * 127) from the two above.
// Each identity holds for every float in its range: tests/cpp/
// quant_arith_check.hip checks them exhaustively on the GPU.
__device__ __forceinline__ float refined_rcp(float a) {
  const float r0 = __builtin_amdgcn_rcpf(a);
  return __builtin_fmaf(__builtin_fmaf(-a, r0, 1.0f), r0, r0);
}
__device__ __forceinline__ float markstein_div(float x, float b, float r) {
  const float q0 = x * r;
  return __builtin_fmaf(__builtin_fmaf(-q0, b, x), r, q0);
}
__device__ __forceinline__ int round_code(float t) {
#pragma clang fp contract(off)
  return static_cast<int>(t + __builtin_copysignf(0.49999997f, t));
}

// The Q8 code of x in a block with maximum amax, given r = RN(1/amax):
// roundf(RN(RN(x/amax) * 127)), the reference's float formula. Contraction is
// off: fused into one FMA, the product and the rounding add skip the rounding
// of the product, and a quotient just below a half (x = 1, amax = 254:
// 0.49999999814 -> RN 0.5 -> code 1) truncates to the code below.
__device__ __forceinline__ int q8_code(float x, float amax, float r) {
#pragma clang fp contract(off)
  const float t = markstein_div(x, amax, r) * 127.0f;
  return static_cast<int>(t + __builtin_copysignf(0.49999997f, t));
}

// Q4_K piece j (0..3): the 32 qs bytes 32j..32j+31, whose low nibbles are
// sub-block 2j and high nibbles sub-block 2j+1, plus the header.
struct Q4KPiece {
  u32x4 head, q0, q1;
};

// Q6_K piece p (0..3) of half h = p/2, parity r = p%2: ql bytes 64h+32r..+31
// (low nibbles: group r, high nibbles: group r+2 of the half), the half's 32
// qh bytes (bits 2g..2g+1 of group g), the scale pairs of both groups and d.
// Q6_K superblocks sit at 210*s, so odd ones start 2 bytes off a dword;
// 16-byte loads at 2-byte alignment run far slower than dword-aligned ones,
// so ql/qh loads start on the dword boundary at or below the field (36 bytes
// cover the 32 field bytes) and v_alignbit realigns in registers.
struct Q6KPiece {
  u32x4 l0, l1, h0, h1;
  uint32_t l2, h2;   // the dwords after l1 / h1
  uint32_t sc_a;     // scales[8h+2r], scales[8h+2r+1] (group r)
  uint32_t sc_b;     // scales[8h+2r+4], scales[8h+2r+5] (group r+2)
  uint32_t d_bits;   // d (2-byte load: a dword could pass the superblock's end)
  uint32_t shift;    // field misalignment in bits: 0 or 16
};

// Q8 activation blocks in LDS, addressed through 32-bit local pointers. (With
// generic pointers the compiler formed 64-bit LDS addresses whose unused high
// half was some other register, and then waited for that register's pending
// global load before the LDS read: a false dependency that serialised the
// weight stream.)
typedef __attribute__((address_space(3))) qk_q8_block lds_q8_block;
typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) u32x2 lds_u32x2;

__device__ __forceinline__ XFrag load_x(const lds_q8_block* xb) {
  const lds_u32x4* p = reinterpret_cast<const lds_u32x4*>(xb);
  XFrag f;
  f.c0 = p[0];  // codes 0..15
  f.c1 = p[1];  // codes 16..31
  f.rec = p[2];  // scale, scaled_sum, neg32_sum_lo, neg32_sum_hi
  return f;
}

__device__ __forceinline__ Q4KPiece load_q4k_piece(const uint8_t* __restrict__ sb, uint32_t j) {
  Q4KPiece f;
  f.head = load16(sb);  // d, dmin, scales[0..11]
  const uint8_t* qs = sb + 16 + 32 * j;
  f.q0 = load16(qs);
  f.q1 = load16(qs + 16);
  return f;
}

// Every byte read lies inside the superblock: the ql run ends at most at
// byte 131 from the dword base, qh at 195, the scale pairs at 207, d at 209.
__device__ __forceinline__ Q6KPiece load_q6k_piece(const uint8_t* __restrict__ sb, uint32_t p) {
  const uint32_t h = p >> 1, r = p & 1u;
  const uint32_t mis = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(sb)) & 3u;  // 0 or 2
  const uint8_t* base = sb - mis;  // dword-aligned
  const uint8_t* ql = base + 64 * h + 32 * r;
  const uint8_t* qh = base + 128 + 32 * h;
  Q6KPiece f;
  f.l0 = load16_a4(ql);
  f.l1 = load16_a4(ql + 16);
  f.l2 = load_u32(ql + 32);
  f.h0 = load16_a4(qh);
  f.h1 = load16_a4(qh + 16);
  f.h2 = load_u32(qh + 32);
  const uint8_t* sc = sb + 192 + 8 * h + 2 * r;  // 2-byte aligned
  f.sc_a = load_u16(sc);
  f.sc_b = load_u16(sc + 4);
  f.d_bits = load_u16(sb + 208);
  f.shift = 8 * mis;
  return f;
}

// Q4_K piece j against the Q8 blocks of sub-blocks 2j (xa) and 2j+1 (xb):
// per sub-block xs*(d*sc*dot) - dmin*m*(xs*sum(codes)), the sub-blocks' terms
// of the reference's per-superblock sum (src/cuda/matmul.cu:24-54).
__device__ __forceinline__ float dot_q4k_piece(const Q4KPiece& w, const XFrag& xa,
                                               const XFrag& xb, uint32_t j) {
  constexpr uint32_t kNib = 0x0F0F0F0Fu;
  const uint32_t q[8] = {w.q0.x, w.q0.y, w.q0.z, w.q0.w, w.q1.x, w.q1.y, w.q1.z, w.q1.w};
  const uint32_t ca[8] = {xa.c0.x, xa.c0.y, xa.c0.z, xa.c0.w, xa.c1.x, xa.c1.y, xa.c1.z, xa.c1.w};
  const uint32_t cb[8] = {xb.c0.x, xb.c0.y, xb.c0.z, xb.c0.w, xb.c1.x, xb.c1.y, xb.c1.z, xb.c1.w};
  int dot_a = 0, dot_b = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    dot_a = dot4(q[i] & kNib, ca[i], dot_a);
    dot_b = dot4((q[i] >> 4) & kNib, cb[i], dot_b);
  }
  int sc_a, m_a, sc_b, m_b;
  scale_min_k4(2 * j, w.head.y, w.head.z, w.head.w, sc_a, m_a);
  scale_min_k4(2 * j + 1, w.head.y, w.head.z, w.head.w, sc_b, m_b);
  const float d = half_bits_to_float(w.head.x & 0xFFFFu);
  const float dmin = half_bits_to_float(w.head.x >> 16);
  const f32x4 ra = __builtin_bit_cast(f32x4, xa.rec);
  const f32x4 rb = __builtin_bit_cast(f32x4, xb.rec);
  // |sc*dot| <= 63*32*15*127 < 2^24, so the integer products convert exactly.
  const float main_a = d * static_cast<float>(__mul24(sc_a, dot_a));
  const float main_b = d * static_cast<float>(__mul24(sc_b, dot_b));
  return (main_a * ra.x - (dmin * static_cast<float>(m_a)) * ra.y) +
         (main_b * rb.x - (dmin * static_cast<float>(m_b)) * rb.y);
}

// A Q6_K piece unpacked: the 6-bit codes of group r (a) and group r+2 (b) of
// its half as bytes (32 each), the four int8 sub-block scales and d. Unpacking
// needs no activations, so a kernel can do it ahead of them.
struct Q6KCodes {
  uint32_t a[8], b[8];
  uint32_t sc;  // bytes: scale of a's first 16, a's last 16, b's first 16, b's last 16
  float d;
};

// (a & mask) | (b & ~mask) in one instruction (the compiler's own pattern
// match misses it once known-bits analysis has narrowed b's mask).
__device__ __forceinline__ uint32_t bit_insert(uint32_t mask, uint32_t a, uint32_t b) {
  uint32_t r;
  asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(r) : "s"(mask), "v"(a), "v"(b));
  return r;
}

// q = ((ql >> 4*(g/2)) & 15) | ((qh >> 2g) & 3) << 4 (src/cuda/matmul.cu:71-79).
// The realignment of a 2-byte-aligned superblock (shift 16) rides in the
// funnel shifts: la = the aligned ql dword (low nibbles: group r), lb = it
// shifted down by 4 (high nibbles: group r+2), qs = the aligned qh dword
// shifted down by 2r and masked to bits 0-1 (group r) and 4-5 (group r+2) of
// every byte; two bit-field inserts form the codes. Bits shifted in from the
// next dword land only in masked-off positions. 7 VALU per 8 codes.
__device__ __forceinline__ Q6KCodes unpack_q6k_piece(const Q6KPiece& w, uint32_t p) {
  const uint32_t r = p & 1u;
  const uint32_t sh = w.shift;  // 0 or 16
  const uint32_t l[9] = {w.l0.x, w.l0.y, w.l0.z, w.l0.w, w.l1.x, w.l1.y, w.l1.z, w.l1.w, w.l2};
  const uint32_t q[9] = {w.h0.x, w.h0.y, w.h0.z, w.h0.w, w.h1.x, w.h1.y, w.h1.z, w.h1.w, w.h2};
  constexpr uint32_t kLo = 0x0F0F0F0Fu, kFields = 0x33333333u;
  Q6KCodes c;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t la = __builtin_amdgcn_alignbit(l[i + 1], l[i], sh);
    const uint32_t lb = __builtin_amdgcn_alignbit(l[i + 1], l[i], sh + 4u);
    const uint32_t qs = __builtin_amdgcn_alignbit(q[i + 1], q[i], sh + 2u * r) & kFields;
    c.a[i] = bit_insert(kLo, la, qs << 4);
    c.b[i] = bit_insert(kLo, lb, qs);
  }
  c.sc = (w.sc_a & 0xFFFFu) | (w.sc_b << 16);
  c.d = half_bits_to_float(w.d_bits);
  return c;
}

// An unpacked Q6_K piece against the Q8 blocks of group r (xa) and group r+2
// (xb) of its half: weight = d*sc*(q-32); the -32 offset enters through the
// Q8 blocks' neg32 sums as the dots' start.
__device__ __forceinline__ float dot_q6k_codes(const Q6KCodes& c, const XFrag& xa, const XFrag& xb) {
  const i32x4 ra = __builtin_bit_cast(i32x4, xa.rec);
  const i32x4 rb = __builtin_bit_cast(i32x4, xb.rec);
  const uint32_t ca[8] = {xa.c0.x, xa.c0.y, xa.c0.z, xa.c0.w, xa.c1.x, xa.c1.y, xa.c1.z, xa.c1.w};
  const uint32_t cb[8] = {xb.c0.x, xb.c0.y, xb.c0.z, xb.c0.w, xb.c1.x, xb.c1.y, xb.c1.z, xb.c1.w};
  int a_lo = ra.z, a_hi = ra.w, b_lo = rb.z, b_hi = rb.w;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    if (i < 4) {
      a_lo = dot4(c.a[i], ca[i], a_lo);
      b_lo = dot4(c.b[i], cb[i], b_lo);
    } else {
      a_hi = dot4(c.a[i], ca[i], a_hi);
      b_hi = dot4(c.b[i], cb[i], b_hi);
    }
  }
  auto s8 = [](uint32_t v, int byte) { return static_cast<int>(static_cast<int8_t>((v >> (8 * byte)) & 0xFFu)); };
  // |sc*dot| <= 64*16*32*127 per group, each sum < 2^24: exact in fp32.
  const int isum_a = __mul24(s8(c.sc, 0), a_lo) + __mul24(s8(c.sc, 1), a_hi);
  const int isum_b = __mul24(s8(c.sc, 2), b_lo) + __mul24(s8(c.sc, 3), b_hi);
  return c.d * (__builtin_bit_cast(float, ra.x) * static_cast<float>(isum_a) +
                __builtin_bit_cast(float, rb.x) * static_cast<float>(isum_b));
}

// Q6_K piece p against the Q8 blocks of group r (xa) and group r+2 (xb) of
// its half (src/cuda/matmul.cu:61-84).
__device__ __forceinline__ float dot_q6k_piece(const Q6KPiece& w, const XFrag& xa,
                                               const XFrag& xb, uint32_t p) {
  return dot_q6k_codes(unpack_q6k_piece(w, p), xa, xb);
}

}  // namespace qk
