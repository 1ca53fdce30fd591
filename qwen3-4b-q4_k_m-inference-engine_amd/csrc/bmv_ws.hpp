// Whole-share batched mat-vec on the int8 matrix cores: M = 2..8 activation
// rows (the decode batch of several sequences), for launches whose
// workgroups own at most 16 rows each (one MFMA row group). Replaces quantize
// + project<Q4_K/Q6_K> with gridDim.y = rows (src/cuda/matmul.cu:8-22,
// 86-125, 151-158), which re-reads every weight row once per activation row.
//
// The tile arithmetic is the batched kernel's (bmv.hpp: one
// v_mfma_i32_16x16x64_i8 takes 16 weight rows against a block-diagonal
// activation tile, sub-block and Q8 scales applied in fp32 per tile); what
// differs is how the weights reach it. There each lane loads its own 16
// bytes of a tile straight from memory (16 rows x 64 bytes per load); here
// the load discipline is the whole-share kernel's (gemv_stream.hpp): wave w
// of a part (MODE 1: waves 0-3 gate, 4-7 up) reads rows R*w .. R*w + R of the
// workgroup (R = 16 / waves per part) as one contiguous run with 16-byte
// loads only, all issued at entry behind the activation loads. After the
// activation quantisation each wave copies its chunks into its LDS region, a
// barrier makes the 16-row group visible, and each wave computes the group's
// tiles of its superblock columns [S*w/Wp, S*(w+1)/Wp) from LDS, leaving its
// column sums in LDS; one thread per (row, activation row) then adds the
// waves' sums in order and stores (results do not depend on timing).
//
// Measured on MI355X at M = 8 (12 distinct matrices back to back in a graph):
// attn_output (2560 x 4096 Q4_K, 10 rows per workgroup) 9.7 us against 11.6
// us on the streaming kernel. Larger shares in phases of 16 rows (gate/up:
// 38 rows per workgroup, q/k/v: 26) were slower than the batched and
// streaming kernels (16.5 against 15.6 us, 14.2 against 12.5 us): the tile
// arithmetic is VALU-bound (~180 VALU per tile and lane, ~4.5 us of the
// gate/up launch per CU), and behind a workgroup barrier per phase most of it
// ran after the stream; so this kernel takes one row group only.
#pragma once

#include "bmv.hpp"

namespace qk {

constexpr int kWsJ = 6;         // 16-byte loads per lane
constexpr int kWsXStaged = 8;   // fp32 activation tasks per lane, all staged ahead of the weights
constexpr int kWsQ8Staged = 4;  // Q8-input blocks per lane, all staged

struct BmvWsParams {
  const float* x;         // [M x K] fp32, or null with q8
  const qk_q8_block* q8;  // [M][K/32] pre-quantised input (mode 0)
  float* h;               // mode 1 output [M x N]
  int32_t M, K, S, nseg;
  int32_t stride;  // LDS bytes per activation row of codes (K + 16)
  int32_t reg;     // LDS bytes of one wave's region
  int32_t act;     // LDS bytes of the activation image (16-byte multiple)
  int32_t pad;
  StreamSegment seg[kMaxSegments];
};

// A launch's plan (bmv_ws_plan): workgroups per segment, LDS bytes of a
// wave's region and of the launch.
struct BmvWsPlan {
  int count[kMaxSegments];
  int reg, lds;
};
struct MatvecParams;
bool bmv_ws_plan(const MatvecParams& p, int mode, int cus, int max_lds, BmvWsPlan& plan);

// LDS image (byte offsets):
//   [0, act)                    activations, as the batched kernel lays them out
//   sums at act                 [parts][16][Wp][8] fp32
//   regions after the sums      8 wave regions of `reg` bytes
__host__ __device__ constexpr int bmv_ws_act_bytes(int K) {
  return (bmv_lds_z(K + 16) + 4 * K + 15) / 16 * 16;
}
__host__ __device__ constexpr int bmv_ws_sums_bytes(int parts) { return parts * 16 * (8 / parts) * 8 * 4; }
__host__ __device__ constexpr int bmv_ws_lds_bytes(int K, int parts, int reg) {
  return bmv_ws_act_bytes(K) + bmv_ws_sums_bytes(parts) + 8 * reg;
}
// A wave's region: its R rows (2 of them 2-byte aligned for Q6_K) plus the
// overshoot of its last 16-byte chunk and the 4 bytes a Q6_K field read may
// look past a superblock.
__host__ __device__ constexpr int bmv_ws_reg_bytes(int rows_per_wave, int row_bytes) {
  return (rows_per_wave * row_bytes + 2 + 15 + 15) / 16 * 16;
}

typedef __attribute__((address_space(3))) uint32_t lds_u32_t;

// 16 bytes at a 2-byte aligned LDS address: dwords dw..dw+4 from the dword
// base below, realigned by sh (0 or 16) bits.
__device__ __forceinline__ u32x4 lds16_realign(const lds_u32_t* b, int dw, uint32_t sh) {
  const uint32_t d0 = b[dw], d1 = b[dw + 1], d2 = b[dw + 2], d3 = b[dw + 3], d4 = b[dw + 4];
  return u32x4{__builtin_amdgcn_alignbit(d1, d0, sh), __builtin_amdgcn_alignbit(d2, d1, sh),
               __builtin_amdgcn_alignbit(d3, d2, sh), __builtin_amdgcn_alignbit(d4, d3, sh)};
}

// A lane's tile image from a superblock in LDS: the same fields bmv_load
// reads from memory (Q4_K superblocks are 16-byte aligned in LDS; Q6_K ones
// 2-byte aligned).
__device__ __forceinline__ void ws_tile(Q4Tile& t, const lds_u8* sb, int kq) {
  t.head = *reinterpret_cast<const lds_u32x4*>(sb);
  t.qa = *reinterpret_cast<const lds_u32x4*>(sb + 16 + 16 * kq);
  t.qb = *reinterpret_cast<const lds_u32x4*>(sb + 80 + 16 * kq);
}
__device__ __forceinline__ void ws_tile(Q6Tile& t, const lds_u8* sb, int kq) {
  const uint32_t mis = lds_offset(sb) & 3u;
  const lds_u32_t* b = reinterpret_cast<const lds_u32_t*>(sb - mis);
  const uint32_t sh = 8u * mis;
  t.la = lds16_realign(b, 4 * kq, sh);              // ql[16kq..]
  t.lb = lds16_realign(b, 16 + 4 * kq, sh);         // ql[64+16kq..]
  t.ha = lds16_realign(b, 32 + 4 * (kq & 1), sh);   // qh[16(kq&1)..]
  t.hb = lds16_realign(b, 40 + 4 * (kq & 1), sh);   // qh[32+16(kq&1)..]
  t.sc = lds16_realign(b, 48, sh);                  // scales
  t.d = __builtin_amdgcn_alignbit(b[53], b[52], sh) & 0xFFFFu;  // d at byte 208
}

// Block b of caller-provided Q8 blocks [M][K/32] (its three 16-byte words:
// codes 0..15, codes 16..31, then scale / scale*sum / -32*sum(0..15) /
// -32*sum(16..31)) into the LDS image bmv_quantize_task writes: the same
// codes, the same scale, the same fp32 product scale*sum and the same
// integer offsets. The record is bit cast as a whole vector: a bit cast of
// one subscripted element (rec.y) was compiled as the vector's first element.
__device__ __forceinline__ void bmv_store_block(u32x4 c0, u32x4 c1, u32x4 rec, int b, int bpr, int stride,
                                                lds_u8* codes, lds_f32* xs, lds_f32* xss, lds_f32* xf) {
  const int m = b / bpr, blk = b - m * bpr;
  lds_u8* row = codes + m * stride + 32 * blk;
  *reinterpret_cast<lds_u32x4*>(row) = c0;
  *reinterpret_cast<lds_u32x4*>(row + 16) = c1;
  const f32x4 rf = __builtin_bit_cast(f32x4, rec);
  const float scale = rf.x;
  xs[blk * 8 + m] = scale;
  xss[blk * 8 + m] = rf.y;
  lds_i32* xi = reinterpret_cast<lds_i32*>(xf);
  xi[(2 * blk) * 8 + m] = static_cast<int32_t>(rec.z);
  xi[(2 * blk + 1) * 8 + m] = static_cast<int32_t>(rec.w);
}

// One type's path of a workgroup: rows [r0, r0 + nrows) (nrows <= 16) of a
// matrix of rows_seg rows (MODE 1: of gate w0 and up w1).
template <int TYPE, int MODE, bool Q8IN>
__device__ __forceinline__ void bmv_ws_body(const BmvWsParams& p, const uint8_t* w0, const uint8_t* w1,
                                            int rows_seg, int r0, int nrows, float* yout,
                                            unsigned char* lds_raw) {
  constexpr int B = TYPE == QK_TYPE_Q4_K ? kQ4KBytes : kQ6KBytes;
  constexpr int kParts = MODE == 1 ? 2 : 1;
  constexpr int kWp = kBmvWaves / kParts;  // waves per part
  constexpr int kRpw = 16 / kWp;           // rows per wave
  const int K = p.K, M = p.M, S = p.S, stride = p.stride;
  const int tid = static_cast<int>(threadIdx.x);
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int part = wave / kWp, wv = wave % kWp;
  const int row_bytes = S * B;

  // activations first: fp32 tasks of 8 values, or Q8 blocks (all staged:
  // the launcher checks that they fit)
  const int groups8 = K / 8, tasks = M * groups8;
  const int bpr = K / 32, nblocks = M * bpr;
  f32x4 xa[Q8IN ? 1 : kWsXStaged], xb[Q8IN ? 1 : kWsXStaged];
  u32x4 qa[Q8IN ? kWsQ8Staged : 1], qb[Q8IN ? kWsQ8Staged : 1], qr[Q8IN ? kWsQ8Staged : 1];
  if constexpr (Q8IN) {
    const u32x4* src = reinterpret_cast<const u32x4*>(p.q8);
#pragma unroll
    for (int i = 0; i < kWsQ8Staged; ++i) {
      const int b = min(tid + 64 * kBmvWaves * i, nblocks - 1);
      qa[i] = src[3 * b];
      qb[i] = src[3 * b + 1];
      qr[i] = src[3 * b + 2];
    }
  } else {
#pragma unroll
    for (int i = 0; i < kWsXStaged; ++i)
      load_x_group(p.x, M, K, min(tid + 64 * kBmvWaves * i, tasks - 1), xa[i], xb[i]);
  }
  __builtin_amdgcn_sched_barrier(0);

  // the wave's run of rows (an empty run re-reads the first chunk)
  WaveShare<kWsJ> ws;
  {
    const int ra = min(kRpw * wv, nrows), rb = min(kRpw * (wv + 1), nrows);
    ws.part = part;
    ws.sb_a = ra * S;
    ws.sb_b = rb * S;
    issue_share<kWsJ>(ws, part ? w1 : w0, rows_seg, r0, S, B, lane);
  }
  __builtin_amdgcn_sched_barrier(0);

  unsigned char* lds = lds_raw;
  lds_u8* codes = (lds_u8*)(lds);
  lds_f32* xs = (lds_f32*)(lds + bmv_lds_z(stride));
  lds_f32* xss = xs + K / 4;
  lds_f32* xf = xs + K / 2;
  lds_f32* sums = (lds_f32*)(lds + p.act);
  lds_u8* regions = (lds_u8*)(lds + p.act + bmv_ws_sums_bytes(kParts));
  if constexpr (Q8IN) {
#pragma unroll
    for (int i = 0; i < kWsQ8Staged; ++i) {
      const int b = tid + 64 * kBmvWaves * i;
      if (b < nblocks) bmv_store_block(qa[i], qb[i], qr[i], b, bpr, stride, codes, xs, xss, xf);
    }
  } else {
#pragma unroll
    for (int i = 0; i < kWsXStaged; ++i) {
      const int t = tid + 64 * kBmvWaves * i;
      if (t < tasks) bmv_quantize_task(xa[i], xb[i], t, groups8, stride, codes, xs, xss, xf);
    }
  }
  if (tid == 0) *reinterpret_cast<lds_u32x4*>(codes + 8 * stride) = u32x4{0u, 0u, 0u, 0u};

  const int reg_bytes = p.reg;
  {  // the wave's chunks into its region
    lds_u8* reg = regions + wave * reg_bytes;
#pragma unroll
    for (int j = 0; j < kWsJ; ++j) {
      const int off = ws.off(j, lane);
      if (TYPE == QK_TYPE_Q4_K || (off & 15) == 0) {
        *reinterpret_cast<lds_u32x4*>(reg + off) = ws.chunk[j];
      } else {
        lds_u32* d = reinterpret_cast<lds_u32*>(reg + off);
        d[0] = ws.chunk[j].x;
        d[1] = ws.chunk[j].y;
        d[2] = ws.chunk[j].z;
        d[3] = ws.chunk[j].w;
      }
    }
  }
  __syncthreads();

  BmvLane L;
  L.n = lane & 15;
  L.kq = lane >> 4;
  L.zero = static_cast<uint32_t>(8 * stride);
  L.a4_valid = (L.n < 8) == (L.kq < 2);
  L.a4_base = static_cast<uint32_t>((L.n & 7) * stride + 16 * (L.kq & 1));
  L.a6_valid = (L.n >> 2) == L.kq;
  L.a6_base = static_cast<uint32_t>((L.n & 3) * stride + 16 * L.kq);
  // the lane's row (rows past the share redo its last one; their sums are
  // never added) and where its wave put it
  const int ic = min(L.n, nrows - 1);
  const int ra = kRpw * (ic / kRpw);
  const uint32_t o = TYPE == QK_TYPE_Q4_K
                         ? 0u
                         : (static_cast<uint32_t>(r0 + ra) * static_cast<uint32_t>(row_bytes)) & 3u;
  const lds_u8* rowp = regions + (part * kWp + ic / kRpw) * reg_bytes + o + (ic % kRpw) * row_bytes;
  const int s_lo = S * wv / kWp, s_hi = S * (wv + 1) / kWp;
  const BmvCursor c{part, 0, wv, 0, 0, 0};
  if constexpr (TYPE == QK_TYPE_Q4_K) {
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int s = s_lo; s < s_hi; ++s) {
      Q4Tile t;
      ws_tile(t, rowp + s * B, L.kq);
      bmv_tile(t, s, L, stride, codes, xs, xss, acc);
    }
    bmv_flush(acc, c, L, 1, kWp, sums);
  } else {
    auto run = [&](auto mh) {
      constexpr int MH = decltype(mh)::value;
      f32x4 acc[2] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
      for (int s = s_lo; s < s_hi; ++s) {
        Q6Tile t;
        ws_tile(t, rowp + s * B, L.kq);
        bmv_tile<MH>(t, s, L, stride, codes, xs, xf, acc);
      }
      bmv_flush<MH>(acc, c, L, 1, kWp, sums);
    };
    if (M > 4) run(std::integral_constant<int, 2>{});
    else run(std::integral_constant<int, 1>{});
  }
  __syncthreads();

  // row totals: the waves' column sums added in wave order; one thread per
  // (activation row, row)
  for (int idx = tid; idx < nrows * M; idx += 64 * kBmvWaves) {
    const int m = idx / nrows, row = idx - m * nrows;
    const lds_f32* pa = sums + row * kWp * 8 + m;
    float a = 0.0f;
#pragma unroll
    for (int rr = 0; rr < kWp; ++rr) a += pa[rr * 8];
    if constexpr (MODE == 0) {
      yout[static_cast<int64_t>(m) * rows_seg + r0 + row] = a;
    } else {
      const lds_f32* pb = pa + 16 * kWp * 8;
      float b = 0.0f;
#pragma unroll
      for (int rr = 0; rr < kWp; ++rr) b += pb[rr * 8];
      p.h[static_cast<int64_t>(m) * rows_seg + r0 + row] = (a / (1.0f + expf(-a))) * b;
    }
  }
}

// TYPE: QK_TYPE_Q4_K or QK_TYPE_Q6_K, or 0 for a launch of both types (each
// workgroup takes its segment's type).
template <int TYPE, int MODE, bool Q8IN>
__global__ __launch_bounds__(64 * kBmvWaves) void bmv_ws_kernel(const BmvWsParams p) {
  extern __shared__ __align__(16) unsigned char lds_raw[];
#pragma unroll
  for (int j = 0; j < kMaxSegments; ++j)
    asm volatile("" ::"s"(p.seg[j].w), "s"(p.seg[j].y), "s"(p.seg[j].rows), "s"(p.seg[j].type),
                 "s"(p.seg[j].wg_begin), "s"(p.seg[j].per), "s"(p.seg[j].rem), "s"(p.seg[j].pad));
  asm volatile("" ::"s"(p.x), "s"(p.q8), "s"(p.h), "s"(p.M), "s"(p.K), "s"(p.S), "s"(p.nseg), "s"(p.stride),
               "s"(p.reg), "s"(p.act), "s"(p.pad));
  __builtin_amdgcn_sched_barrier(0);
  const int wg = static_cast<int>(blockIdx.x), nseg = p.nseg;
  const int j = (nseg > 1 && wg >= p.seg[1].wg_begin) + (nseg > 2 && wg >= p.seg[2].wg_begin) +
                (nseg > 3 && wg >= p.seg[3].wg_begin);
  auto pick = [j](auto f0, auto f1, auto f2, auto f3) {
    return j == 0 ? f0 : j == 1 ? f1 : j == 2 ? f2 : f3;
  };
  const int type = pick(p.seg[0].type, p.seg[1].type, p.seg[2].type, p.seg[3].type);
  const int rows = pick(p.seg[0].rows, p.seg[1].rows, p.seg[2].rows, p.seg[3].rows);
  const int g = wg - pick(p.seg[0].wg_begin, p.seg[1].wg_begin, p.seg[2].wg_begin, p.seg[3].wg_begin);
  const int per = pick(p.seg[0].per, p.seg[1].per, p.seg[2].per, p.seg[3].per);
  const int rem = pick(p.seg[0].rem, p.seg[1].rem, p.seg[2].rem, p.seg[3].rem);
  float* yout = pick(p.seg[0].y, p.seg[1].y, p.seg[2].y, p.seg[3].y);
  const uint8_t* w0 = pick(p.seg[0].w, p.seg[1].w, p.seg[2].w, p.seg[3].w);
  const uint8_t* w1 = MODE == 1 ? p.seg[1].w : w0;
  const int r0 = g * per + min(g, rem);
  const int nrows = per + (g < rem ? 1 : 0);
  if constexpr (TYPE == 0) {
    if (type == QK_TYPE_Q4_K)
      bmv_ws_body<QK_TYPE_Q4_K, MODE, Q8IN>(p, w0, w1, rows, r0, nrows, yout, lds_raw);
    else
      bmv_ws_body<QK_TYPE_Q6_K, MODE, Q8IN>(p, w0, w1, rows, r0, nrows, yout, lds_raw);
  } else {
    bmv_ws_body<TYPE, MODE, Q8IN>(p, w0, w1, rows, r0, nrows, yout, lds_raw);
  }
}

using BmvWsKernel = void (*)(BmvWsParams);

// The instantiations (bmv_ws.hip); type 0 is the mixed launch. Null when
// there is no such kernel.
BmvWsKernel bmv_ws_kernel_for(int type, int mode, bool q8in);

}  // namespace qk
