// Batched mat-vec on the int8 matrix cores: M = 2..8 activation rows (the
// decode batch of several sequences), fp32 activations quantised in the
// kernel. Replaces quantize + project<Q4_K/Q6_K> with gridDim.y = rows
// (src/cuda/matmul.cu:8-22, 86-125, 151-158), which re-reads every weight row
// once per activation row.
//
// With integer dots on the vector ALU every lane needs the activation bytes
// that match its weights, so an M-row launch reads M activation fragments
// from LDS per weight piece (96 bytes per 64 weights per row): at M = 8 the
// LDS, not HBM, bounds it. Here one v_mfma_i32_16x16x64_i8 takes 16 weight
// rows (B columns) against an activation tile (A rows) that all 16 rows
// share. Sub-block scales (32 weights for Q4_K, 16 for Q6_K) and the Q8
// block scales (32 activations) vary along k, so each MFMA spans exactly the
// sub-blocks whose products it keeps apart: its A tile is block-diagonal.
//   Q4_K: k 0..31 = sub-block j1, k 32..63 = j2 (the low or high nibbles of
//         64 qs bytes); A rows 0..7 = activation rows 0..7 against j1, rows
//         8..15 = the same rows against j2, zero elsewhere.
//   Q6_K: k = 4 sub-blocks of 16 (one nibble of 64 ql bytes with their qh
//         bit pairs); A rows 4b..4b+3 = 4 activation rows against sub-block
//         b; a second MFMA on the same B takes activation rows 4..7.
// Lane l holds A[l%16][16(l/16)..+16], B[16(l/16)..+16][l%16] and receives
// C[4(l/16)+i][l%16], i < 4 (probed on gfx950), so lane (n, kq) = (l%16, l/16)
// loads the 16 weight bytes of row n for k-quarter kq straight from memory,
// and its four integer results belong to one sub-block and four activation
// rows: they are scaled by that sub-block's scale and the rows' Q8 scales in
// fp32 (Q4_K: d*sc*xs*dot - dmin*m*xs*sum(codes); Q6_K: d*sc*xs*(dot - 32
// sum(codes)), src/cuda/matmul.cu:24-84).
//
// A workgroup (one per CU) owns a contiguous range of rows of one segment;
// its rows are cut into groups of 16 and each group's superblock columns
// into `ranges` runs. Work units (part, group, run) are dealt to the waves in
// contiguous blocks; a wave streams its units' tiles (16 rows x one
// superblock) through a ring of P register buffers, P tiles ahead, so
// memory stays busy while earlier tiles are computed. Each unit's sums go to
// LDS; after a barrier one thread per (row, activation row) adds the runs in
// order and stores (results do not depend on timing).
#pragma once

#include <type_traits>

#include "gemv_stream.hpp"

namespace qk {

// 8 waves of up to 256 registers each: deep per-wave tile rings without
// spills (a scratch reload counts in the same vmcnt as the weight loads, so
// one spill in the loop would serialise the stream)
constexpr int kBmvWaves = 8;    // waves per workgroup (one workgroup per CU)
// activation tasks per lane whose loads are issued before the weights (held
// in registers with the first tiles during the quantisation)
constexpr int kBmvXStaged4 = 5;
constexpr int kBmvXStaged6 = 5;
constexpr int kBmvP4 = 6;       // Q4_K tiles in flight per wave
constexpr int kBmvP6 = 4;       // Q6_K tiles in flight per wave
constexpr int kBmvP6Mixed = 3;  // Q6_K tiles in flight in a launch with both types
// Q8 blocks of h one workgroup may complete (M activation rows each, a quad
// per block row): the launcher checks blocks * M * 4 <= threads.
constexpr int kBmvMaxCloseBlocks = 16;

struct BmvParams {
  const float* x;       // [M x K]
  float* h;             // mode 1 output [M x N]
  qk_q8_block* hq;      // mode 1, optional: Q8 of h [M][N/32], formed in the launch
  uint32_t* arrive;     // with hq: per-block arrival counters [N/32], zero between launches
  int32_t M, K, S, nseg;
  int32_t stride;      // LDS bytes per activation row of codes (K + 16)
  int32_t ranges;      // superblock runs per row group
  int32_t groups_max;  // row groups of the largest workgroup share
  int32_t pad;
  StreamSegment seg[kMaxSegments];
};

// LDS image (byte offsets; K a multiple of 256):
//   codes [8][stride] int8         at 0 (rows m >= M are never written)
//   zero  16 bytes                 at 8*stride
//   xs    [K/32][8] fp32 Q8 scale  at Z = 8*stride + 16
//   xss   [K/32][8] fp32 scale*sum(codes)          at Z + K
//   xf    [K/16][8] int32 -32*(sum of 16 codes)    at Z + 2K (the Q6_K offset,
//                                                  the MFMA's accumulator input)
//   sums  [parts][groups_max][16][ranges][8] fp32  at Z + 4K
// Rows m >= M of every array are left unwritten: they feed only results for
// activation rows that are never stored.
__host__ __device__ constexpr int bmv_lds_z(int stride) { return 8 * stride + 16; }
__host__ __device__ constexpr int bmv_lds_bytes(int K, int stride, int parts, int groups, int ranges) {
  return bmv_lds_z(stride) + 4 * K + parts * groups * 16 * ranges * 32;
}

typedef __attribute__((address_space(3))) f32x4 lds_f32x4;

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i32x4 lds_i32x4;
typedef __attribute__((address_space(3))) int32_t lds_i32;

// Task t (8 activations of the [M][K] stream): codes to row t / (K/8), the
// block's scales by lane 0 of its quad.
__device__ __forceinline__ void bmv_quantize_task(f32x4 a, f32x4 b, int t, int groups, int stride,
                                                  lds_u8* codes, lds_f32* xs, lds_f32* xss, lds_f32* xf) {
  const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  const Q8Quarter q = quantize_quarter(v);
  const int m = t / groups, k0 = 8 * (t - m * groups);
  *reinterpret_cast<lds_u32x2*>(codes + m * stride + k0) = u32x2{q.lo, q.hi};
  if ((t & 3) == 0) {
    const int blk = k0 >> 5;
    xs[blk * 8 + m] = q.scale;
    xss[blk * 8 + m] = q.scale * static_cast<float>(q.pair + q.other);
    lds_i32* xi = reinterpret_cast<lds_i32*>(xf);
    xi[(2 * blk) * 8 + m] = -32 * q.pair;
    xi[(2 * blk + 1) * 8 + m] = -32 * q.other;
  }
}

// A lane's register image of one tile (16 rows x one superblock).
struct Q4Tile {
  u32x4 head, qa, qb;  // d, dmin, scales; qs[16kq..+16]; qs[64+16kq..+16]
};
struct Q6Tile {
  u32x4 la, lb, ha, hb, sc;  // ql[16kq..], ql[64+16kq..], qh[16(kq&1)..], qh[32+16(kq&1)..], scales
  uint32_t d;
};

template <int TYPE>
using BmvTile = typename std::conditional<TYPE == QK_TYPE_Q4_K, Q4Tile, Q6Tile>::type;

// Loads of a tile: sb = this lane's row's superblock (16-byte aligned for
// Q4_K, 2-byte for Q6_K); every byte read lies inside the superblock.
__device__ __forceinline__ void bmv_load(Q4Tile& t, const uint8_t* sb, int kq) {
  t.head = load16(sb);
  t.qa = load16(sb + 16 + 16 * kq);
  t.qb = load16(sb + 80 + 16 * kq);
}
__device__ __forceinline__ void bmv_load(Q6Tile& t, const uint8_t* sb, int kq) {
  t.la = load16_a2(sb + 16 * kq);
  t.lb = load16_a2(sb + 64 + 16 * kq);
  t.ha = load16_a2(sb + 128 + 16 * (kq & 1));
  t.hb = load16_a2(sb + 160 + 16 * (kq & 1));
  t.sc = load16_a2(sb + 192);
  t.d = load_u16(sb + 208);
}

__device__ __forceinline__ i32x4 mfma_i8(i32x4 a, u32x4 b, i32x4 c = i32x4{0, 0, 0, 0}) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, __builtin_bit_cast(i32x4, b), c, 0, 0, 0);
}

__device__ __forceinline__ i32x4 lds_read_i32x4(const lds_u8* base, uint32_t off) {
  return *reinterpret_cast<const lds_i32x4*>(base + off);
}
__device__ __forceinline__ f32x4 lds_read_f32x4(const lds_f32* p) {
  return *reinterpret_cast<const lds_f32x4*>(p);
}

// Per-lane constants of the tile computation.
struct BmvLane {
  int n, kq;
  uint32_t a4_base;   // Q4_K A: this lane's activation row and k-quarter, or the zero line
  bool a4_valid;
  uint32_t a6_base;   // Q6_K A (activation rows 0..3; rows 4..7 add 4*stride)
  bool a6_valid;
  uint32_t zero;
};

// Q4_K tile at superblock column s: acc[i] += row n's dot for activation row
// 4*(kq&1)+i over the sub-blocks of set kq>>1 (the other set sits in lane l^32).
__device__ __forceinline__ void bmv_tile(const Q4Tile& t, int s, const BmvLane& L, int stride,
                                         const lds_u8* codes, const lds_f32* xs, const lds_f32* xss,
                                         f32x4& acc) {
  const int khi = L.kq >> 1, klo = L.kq & 1;
  i32x4 c[4];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
#pragma unroll
    for (int nib = 0; nib < 2; ++nib) {
      const int j = 4 * h + nib + 2 * khi;  // this lane's sub-block (A side and C side)
      const uint32_t aoff = L.a4_valid ? L.a4_base + 256 * s + 32 * j : L.zero;
      const u32x4 q = h ? t.qb : t.qa;
      const u32x4 bq = nib ? ((q >> 4) & 0x0F0F0F0Fu) : (q & 0x0F0F0F0Fu);
      c[2 * h + nib] = mfma_i8(lds_read_i32x4(codes, aoff), bq);
    }
  }
  const uint32_t s0 = t.head.y, s1 = t.head.z, s2 = t.head.w;
  f32x4 mainv = {0.0f, 0.0f, 0.0f, 0.0f}, minv = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int h = 0; h < 2; ++h) {
#pragma unroll
    for (int nib = 0; nib < 2; ++nib) {
      const int j = 4 * h + nib + 2 * khi;
      // 6-bit (scale, min) of sub-block j (get_scale_min_k4, src/cuda/embedding.cu:20-23)
      const uint32_t o = 8u * static_cast<uint32_t>(nib + 2 * khi);
      uint32_t sc, mn;
      if (h == 0) {
        sc = ubfe(s0, o, 6);
        mn = ubfe(s1, o, 6);
      } else {
        sc = ubfe(s2, o, 4) | (ubfe(s0, o + 6, 2) << 4);
        mn = ubfe(s2, o + 4, 4) | (ubfe(s1, o + 6, 2) << 4);
      }
      const float scf = static_cast<float>(sc);
      const float mf = static_cast<float>(mn);
      const f32x4 x4 = lds_read_f32x4(xs + (8 * s + j) * 8 + 4 * klo);
      const f32x4 y4 = lds_read_f32x4(xss + (8 * s + j) * 8 + 4 * klo);
      const i32x4 ci = c[2 * h + nib];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        mainv[i] = __builtin_fmaf(static_cast<float>(ci[i]), x4[i] * scf, mainv[i]);
        minv[i] = __builtin_fmaf(mf, y4[i], minv[i]);
      }
    }
  }
  const float d = half_bits_to_float(t.head.x & 0xFFFFu);
  const float dmin = half_bits_to_float(t.head.x >> 16);
#pragma unroll
  for (int i = 0; i < 4; ++i) acc[i] = __builtin_fmaf(-dmin, minv[i], __builtin_fmaf(d, mainv[i], acc[i]));
}

// Q6_K tile at superblock column s: acc[mh][i] += row n's dot for activation
// row 4*mh+i over the sub-blocks 8h+4nib+kq (the other kq in lanes l^16, l^32).
template <int MH>
__device__ __forceinline__ void bmv_tile(const Q6Tile& t, int s, const BmvLane& L, int stride,
                                         const lds_u8* codes, const lds_f32* xs, const lds_f32* xf,
                                         f32x4 (&acc)[2]) {
  const int khi = L.kq >> 1;
  // qh bit pair of group g = 2nib + khi moved to bits 4-5 of each byte
  const uint32_t sh0 = 28u + 2u * static_cast<uint32_t>(khi), sh1 = 2u * static_cast<uint32_t>(khi);
  f32x4 accsb[2] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
#pragma unroll
  for (int h = 0; h < 2; ++h) {
#pragma unroll
    for (int nib = 0; nib < 2; ++nib) {
      // 16 codes (ql nibble | qh pair << 4, 0..63; the -32 offset enters
      // as the MFMA's accumulator input -32 * sum(activation codes), so the
      // integer dot is exact): src/cuda/matmul.cu:71-79
      const u32x4 ql = h ? t.lb : t.la;
      const u32x4 qh = h ? t.hb : t.ha;
      const uint32_t sh = nib ? sh1 : sh0;
      u32x4 b;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t lo = nib ? (ql[e] >> 4) & 0x0F0F0F0Fu : ql[e] & 0x0F0F0F0Fu;
        const uint32_t hs = __builtin_amdgcn_alignbit(qh[e], qh[e], sh);
        b[e] = bit_insert(0x30303030u, hs, lo);
      }
      const int sb16 = 8 * h + 4 * nib + L.kq;  // this lane's sub-block
      const float scf = static_cast<float>(static_cast<int8_t>((t.sc[2 * h + nib] >> (8 * L.kq)) & 0xFFu));
      const int blk = 4 * h + 2 * nib + khi;  // its Q8 block
#pragma unroll
      for (int mh = 0; mh < MH; ++mh) {
        const uint32_t aoff = L.a6_valid ? L.a6_base + 4 * mh * stride + 256 * s + 128 * h + 64 * nib : L.zero;
        const i32x4 n4 = lds_read_i32x4(reinterpret_cast<const lds_u8*>(xf), 4u * ((16 * s + sb16) * 8 + 4 * mh));
        const i32x4 ci = mfma_i8(lds_read_i32x4(codes, aoff), b, n4);
        const f32x4 x4 = lds_read_f32x4(xs + (8 * s + blk) * 8 + 4 * mh);
#pragma unroll
        for (int i = 0; i < 4; ++i)
          accsb[mh][i] = __builtin_fmaf(scf, x4[i] * static_cast<float>(ci[i]), accsb[mh][i]);
      }
    }
  }
  const float d = half_bits_to_float(t.d);
#pragma unroll
  for (int mh = 0; mh < MH; ++mh)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[mh][i] = __builtin_fmaf(d, accsb[mh][i], acc[mh][i]);
}

// Position of a wave in its stream of tiles: unit (part, group g, run rr),
// superblock s of the run [s, s_end), tiles left including this one.
struct BmvCursor {
  int part, g, rr, s, s_end, left;
};

// The workgroup's share of one segment and the run split of superblocks.
struct BmvShare {
  const uint8_t* w[2];  // per part (mode 1: gate, up)
  int r0, nrows, groups, S, row_bytes, ranges, run_q, run_r;
  int per, rem;  // the segment's cut: per rows a workgroup, the first rem one more
  __device__ __forceinline__ int run_begin(int rr) const { return rr * run_q + min(rr, run_r); }
};

__device__ __forceinline__ void cursor_seek(BmvCursor& c, const BmvShare& sh, int u) {
  c.rr = u % sh.ranges;
  const int pg = u / sh.ranges;
  c.part = pg / sh.groups;
  c.g = pg - c.part * sh.groups;
  c.s = sh.run_begin(c.rr);
  c.s_end = sh.run_begin(c.rr + 1);
}

__device__ __forceinline__ void cursor_next(BmvCursor& c, const BmvShare& sh) {
  if (c.left > 1) {
    --c.left;
    if (++c.s == c.s_end) {
      if (++c.rr == sh.ranges) {
        c.rr = 0;
        if (++c.g == sh.groups) {
          c.g = 0;
          ++c.part;
        }
      }
      c.s = sh.run_begin(c.rr);
      c.s_end = sh.run_begin(c.rr + 1);
    }
  }
}

// This lane's superblock of the cursor's tile: row min(16g + n, nrows - 1)
// of the share (rows past the share re-read its last row; their results are
// not stored).
template <int B>
__device__ __forceinline__ const uint8_t* bmv_sb(const BmvShare& sh, const BmvCursor& c, int n) {
  const int row = min(16 * c.g + n, sh.nrows - 1);
  return (c.part ? sh.w[1] : sh.w[0]) + static_cast<int64_t>(sh.r0 + row) * sh.row_bytes + c.s * B;
}

// Unit sums into LDS: sums[((part*groups_max + g)*16 + n)*ranges + rr][m].
__device__ __forceinline__ void bmv_flush(const f32x4& acc, const BmvCursor& c, const BmvLane& L,
                                          int groups_max, int ranges, lds_f32* sums) {
  f32x4 v;
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = swap32_sum(acc[i]);  // both sub-block sets
  if (L.kq < 2)
    *reinterpret_cast<lds_f32x4*>(sums + (((c.part * groups_max + c.g) * 16 + L.n) * ranges + c.rr) * 8 +
                                  4 * L.kq) = v;
}
template <int MH>
__device__ __forceinline__ void bmv_flush(const f32x4 (&acc)[2], const BmvCursor& c, const BmvLane& L,
                                          int groups_max, int ranges, lds_f32* sums) {
  f32x4 v[2];
#pragma unroll
  for (int mh = 0; mh < MH; ++mh)
#pragma unroll
    for (int i = 0; i < 4; ++i) v[mh][i] = swap16_sum(swap32_sum(acc[mh][i]));  // all four kq
  if (L.kq == 0) {
    lds_f32* p = sums + (((c.part * groups_max + c.g) * 16 + L.n) * ranges + c.rr) * 8;
#pragma unroll
    for (int mh = 0; mh < MH; ++mh) *reinterpret_cast<lds_f32x4*>(p + 4 * mh) = v[mh];
  }
}

// One type's share: the tile stream of this wave, then (after the caller's
// barrier) nothing; the caller forms the row totals.
template <int TYPE, int P, int MH>
__device__ __forceinline__ void bmv_stream(const BmvShare& sh, BmvCursor lc, const BmvLane& L, int stride,
                                           int groups_max, const lds_u8* codes, const lds_f32* xs,
                                           const lds_f32* xss, const lds_f32* xf, lds_f32* sums,
                                           BmvTile<TYPE> (&buf)[P], BmvCursor cc) {
  constexpr int B = TYPE == QK_TYPE_Q4_K ? kQ4KBytes : kQ6KBytes;
  using Acc = typename std::conditional<TYPE == QK_TYPE_Q4_K, f32x4, f32x4[2]>::type;
  Acc acc;
  auto clear = [&]() {
    if constexpr (TYPE == QK_TYPE_Q4_K) {
      acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    } else {
      acc[0] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      acc[1] = acc[0];
    }
  };
  clear();
  const int ntiles = cc.left;
  for (int base = 0; base < ntiles; base += P) {
#pragma unroll
    for (int j = 0; j < P; ++j) {
      if (base + j < ntiles) {
        if constexpr (TYPE == QK_TYPE_Q4_K)
          bmv_tile(buf[j], cc.s, L, stride, codes, xs, xss, acc);
        else
          bmv_tile<MH>(buf[j], cc.s, L, stride, codes, xs, xf, acc);
        if (cc.s + 1 == cc.s_end) {  // last tile of the unit
          if constexpr (TYPE == QK_TYPE_Q4_K)
            bmv_flush(acc, cc, L, groups_max, sh.ranges, sums);
          else
            bmv_flush<MH>(acc, cc, L, groups_max, sh.ranges, sums);
          clear();
        }
        cursor_next(cc, sh);
      }
      // refill the buffer P tiles ahead (past the end: the last tile again,
      // from cache), unconditionally so the waits count it
      bmv_load(buf[j], bmv_sb<B>(sh, lc, L.n), L.kq);
      cursor_next(lc, sh);
    }
  }
}

}  // namespace qk
