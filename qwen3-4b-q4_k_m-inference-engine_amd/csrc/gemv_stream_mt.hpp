// Whole-share mat-vec for MT = 4 or 8 activation rows (batched decode, M = 2..8):
// the M = 1 kernel's loading (gemv_stream.hpp) with a compute layout that
// reuses every activation fragment across 16 weight rows.
//
// Replaces project<Q4_K/Q6_K> with gridDim.y = rows (src/cuda/matmul.cu:151-158)
// for the decode batch. The streaming kernel spends most of an M = 8 launch
// quantising the activations (every CU quantises all M*K of them, a task per
// lane at a time) and reads each activation fragment from LDS once per weight
// piece. Here:
//   1. all 16 waves stage up to 4 activation tasks each, issue their weight
//      loads (each wave a contiguous run of whole rows of the workgroup's
//      share, 16-byte loads only), quantise, and copy their chunks to LDS;
//   2. after a barrier, work units (part, group of 16 rows, range of
//      superblock columns) are dealt to the waves: lane = (row of the group,
//      piece), and for each column s the lanes unpack their piece once and
//      take its dot with the MT activation rows' Q8 blocks of column s, which
//      all 16 rows of the group share (LDS broadcasts);
//   3. per-unit sums go to LDS; after a barrier one thread per (row, m) adds
//      the ranges in order and stores (mode 1: SiLU(gate) * up).
#pragma once

#include "gemv_stream.hpp"

namespace qk {

constexpr int kMtXStaged = 4;  // activation tasks per lane: MT * K / 8 <= 4096

struct StreamMtParams {
  const float* x;  // [M x K]
  float* h;        // mode 1 output [M x N]
  int32_t M, K, S, nseg;
  int32_t region;     // LDS bytes of a wave's weight region (a multiple of 16)
  int32_t sums_stride;  // floats of unit sums per part: rows_max * ranges_max * MT
  StreamSegment seg[kMaxSegments];
};

template <int MT>
struct MtStage {
  f32x4 a[kMtXStaged], b[kMtXStaged];
};

// Consumption after the activations are in LDS: chunks to LDS, a barrier,
// the work units, a barrier, the row totals.
template <int MT, int TYPE, int J, int MODE>
__device__ __forceinline__ void stream_mt_consume(const u32x4 (&chunk)[J], const int (&off)[J],
                                                  int o, int rpw, int r0, int nrows, int S, int M,
                                                  int rows_seg, int region, int sums_stride,
                                                  global_f32* y, global_f32* h,
                                                  const lds_q8_block* xq, lds_u8* wlds,
                                                  lds_f32* sums) {
  constexpr int B = TYPE == QK_TYPE_Q4_K ? kQ4KBytes : kQ6KBytes;
  constexpr int kParts = MODE == 1 ? 2 : 1;
  constexpr int kWpp = kStreamWaves / kParts;
  const int lane = static_cast<int>(threadIdx.x & 63u);
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  lds_u8* reg = wlds + wave * region;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    if (TYPE == QK_TYPE_Q4_K || (off[j] & 15) == 0) {
      *reinterpret_cast<lds_u32x4*>(reg + off[j]) = chunk[j];
    } else {
      lds_u32* d = reinterpret_cast<lds_u32*>(reg + off[j]);
      d[0] = chunk[j].x;
      d[1] = chunk[j].y;
      d[2] = chunk[j].z;
      d[3] = chunk[j].w;
    }
  }
  __syncthreads();

  // Units: part x group of 16 rows x range of columns, ranges enough for
  // about 16 units. Row r of a part sits in the region of wave
  // part*kWpp + r/rpw, (r % rpw) rows after that wave's first row, whose
  // superblock 0 starts o(r0 + first) bytes into the region (0 or 2).
  const int groups = (nrows + 15) >> 4;
  const int ranges = min(S, max(1, (kStreamWaves + kParts * groups - 1) / (kParts * groups)));
  const int units = kParts * groups * ranges;
  const int row_bytes = S * B;
  const uint32_t pc = static_cast<uint32_t>(lane) & 3u;
  const int blk_a = piece_block_a(pc, TYPE), blk_step = piece_block_step(TYPE);
  for (int u = wave; u < units; u += kStreamWaves) {
    const int part = u / (groups * ranges);
    const int g = (u / ranges) % groups;
    const int rr = u % ranges;
    const int row = min(g * 16 + (lane >> 2), nrows - 1);  // lanes past the rows redo the last row
    const int owner = part * kWpp + row / rpw;
    const int first = (row / rpw) * rpw;  // the owner's first row
    const int o_owner = (o + first * (row_bytes & 3)) & 3;  // the owner's run offset
    const lds_u8* rowp = wlds + owner * region + o_owner + (row - first) * row_bytes;
    const int s0 = S * rr / ranges, s1 = S * (rr + 1) / ranges;
    float acc[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[m] = 0.0f;
    const lds_u8* sbp = rowp + s0 * B;
    for (int s = s0; s < s1; ++s, sbp += B) {
      const lds_q8_block* xs = xq + ((s * 8 + blk_a) & 0xFFFF);
      if constexpr (TYPE == QK_TYPE_Q4_K) {
        const Q4KPiece f = lds_q4k_piece(sbp, pc);
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          const lds_q8_block* xr = xs + m * S * 8;
          acc[m] += dot_q4k_piece(f, load_x(xr), load_x(xr + blk_step), pc);
        }
      } else {
        // the piece unpacked once for all MT rows (the same arithmetic as
        // dot_q6k_piece per row)
        const Q6KCodes cd = unpack_q6k_piece(lds_q6k_piece(sbp, pc), pc);
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          const lds_q8_block* xr = xs + m * S * 8;
          acc[m] += dot_q6k_codes(cd, load_x(xr), load_x(xr + blk_step));
          // rows in pairs: the pair's sums are formed before the next rows'
          // LDS reads (IR-level code motion otherwise hoists every row's reads)
          if (MT > 2 && (m & 1)) {
            asm volatile("" ::"v"(acc[m - 1]), "v"(acc[m]) : "memory");
            __builtin_amdgcn_sched_barrier(0);
          }
        }
      }
    }
    const bool live = pc == 0 && g * 16 + (lane >> 2) < nrows;
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      const float v = add_dpp<0x4E>(add_dpp<0xB1>(acc[m]));
      if (live) sums[part * sums_stride + (row * ranges + rr) * MT + m] = v;
    }
  }
  __syncthreads();

  // Row totals: one thread per (row, m < M), the ranges added in order.
  for (int t = static_cast<int>(threadIdx.x); t < nrows * M; t += 64 * kStreamWaves) {
    const int row = t / M, m = t - row * M;
    float g = 0.0f, v = 0.0f;
    for (int rr = 0; rr < ranges; ++rr) {
      g += sums[(row * ranges + rr) * MT + m];
      if constexpr (MODE == 1) v += sums[sums_stride + (row * ranges + rr) * MT + m];
    }
    if constexpr (MODE == 0) y[static_cast<int64_t>(m) * rows_seg + r0 + row] = g;
    else h[static_cast<int64_t>(m) * rows_seg + r0 + row] = (g / (1.0f + expf(-g))) * v;
  }
}

// TYPE: every segment's weight type (one type per launch: the mixed-type build
// spills registers and ran slower than the streaming kernel).
template <int MT, int TYPE, int J, int MODE>
__global__ __launch_bounds__(64 * kStreamWaves) void stream_mt_kernel(const StreamMtParams p) {
  static_assert(TYPE == QK_TYPE_Q4_K || TYPE == QK_TYPE_Q6_K, "one weight type per launch");
  extern __shared__ __align__(16) unsigned char lds_raw[];
  constexpr int kParts = MODE == 1 ? 2 : 1;
  constexpr int kWpp = kStreamWaves / kParts;
#pragma unroll
  for (int j = 0; j < kMaxSegments; ++j)
    asm volatile("" ::"s"(p.seg[j].w), "s"(p.seg[j].y), "s"(p.seg[j].rows), "s"(p.seg[j].type),
                 "s"(p.seg[j].wg_begin), "s"(p.seg[j].per), "s"(p.seg[j].rem), "s"(p.seg[j].pad));
  asm volatile("" ::"s"(p.x), "s"(p.h), "s"(p.M), "s"(p.K), "s"(p.S), "s"(p.nseg), "s"(p.region),
               "s"(p.sums_stride));
  __builtin_amdgcn_sched_barrier(0);
  const int K = p.K, nseg = p.nseg, M = p.M;
  const int lane = static_cast<int>(threadIdx.x & 63u);
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));

  // activation tasks (8 values each) t = threadIdx.x + 1024 i of the [MT][K] stream
  const int tasks = MT * (K / 8);
  MtStage<MT> st;
#pragma unroll
  for (int i = 0; i < kMtXStaged; ++i) {
    const int t = min(static_cast<int>(threadIdx.x) + 64 * kStreamWaves * i, tasks - 1);
    load_x_group(p.x, M, K, t, st.a[i], st.b[i]);
  }
  __builtin_amdgcn_sched_barrier(0);

  const int wg = static_cast<int>(blockIdx.x);
  const int j = (nseg > 1 && wg >= p.seg[1].wg_begin) + (nseg > 2 && wg >= p.seg[2].wg_begin) +
                (nseg > 3 && wg >= p.seg[3].wg_begin);
  auto pick = [j](auto f0, auto f1, auto f2, auto f3) {
    return j == 0 ? f0 : j == 1 ? f1 : j == 2 ? f2 : f3;
  };
  const uint8_t* w0 = pick(p.seg[0].w, p.seg[1].w, p.seg[2].w, p.seg[3].w);
  float* yout = pick(p.seg[0].y, p.seg[1].y, p.seg[2].y, p.seg[3].y);
  int rows = pick(p.seg[0].rows, p.seg[1].rows, p.seg[2].rows, p.seg[3].rows);
  const int g = wg - pick(p.seg[0].wg_begin, p.seg[1].wg_begin, p.seg[2].wg_begin, p.seg[3].wg_begin);
  const int per = pick(p.seg[0].per, p.seg[1].per, p.seg[2].per, p.seg[3].per);
  const int rem = pick(p.seg[0].rem, p.seg[1].rem, p.seg[2].rem, p.seg[3].rem);
  int r0 = g * per + min(g, rem);
  int nrows = per + (g < rem ? 1 : 0);
  // values used after the barriers held in registers (see stream_matvec_kernel)
  int S = p.S, region = p.region, sums_stride = p.sums_stride, Mr = M;
  float* hout = p.h;
  asm volatile("" : "+s"(S), "+s"(region), "+s"(sums_stride), "+s"(Mr), "+s"(hout), "+s"(yout),
               "+s"(r0), "+s"(nrows), "+s"(rows));

  // This wave's run: rows [first, first + rpw) of its part, as 16-byte chunks
  // from the dword boundary at or below the run (moved back at the matrix
  // end, as in the one-row kernel).
  constexpr int B = TYPE == QK_TYPE_Q4_K ? kQ4KBytes : kQ6KBytes;
  const int rpw = (nrows + kWpp - 1) / kWpp;
  const int part = wave / kWpp;
  const int first = min((wave % kWpp) * rpw, nrows);
  const int wrows = min(rpw, nrows - first);
  const uint8_t* w = MODE == 1 && part ? p.seg[1].w : w0;
  const int64_t row_bytes = static_cast<int64_t>(S) * B;
  const uint8_t* run = w + (r0 + (wrows > 0 ? first : 0)) * row_bytes;
  const int o = static_cast<int>(reinterpret_cast<uintptr_t>(run) & 3u);
  const uint8_t* run4 = run - o;
  const int L = max((o + wrows * static_cast<int>(row_bytes) + 15) >> 4, 1);
  const uint8_t* last = w + ((rows * row_bytes + 3) & ~int64_t{3}) - 16;
  u32x4 chunk[J];
  int off[J];
#pragma unroll
  for (int jj = 0; jj < J; ++jj) {
    const int c = min(lane + 64 * jj, L - 1);
    const uint8_t* a = run4 + 16 * c;
    a = a < last ? a : last;
    off[jj] = static_cast<int>(a - run4);
    chunk[jj] = stream_load16_a4(a);
  }
  __builtin_amdgcn_sched_barrier(0);

  lds_q8_block* xq = (lds_q8_block*)(lds_raw);
  lds_u8* wlds = (lds_u8*)(lds_raw) + MT * S * 8 * static_cast<int>(sizeof(qk_q8_block));
  lds_f32* sums = reinterpret_cast<lds_f32*>(wlds + kStreamWaves * region);
  {
    const int groups = K / 8;
#pragma unroll
    for (int i = 0; i < kMtXStaged; ++i) {
      const int t = static_cast<int>(threadIdx.x) + 64 * kStreamWaves * i;
      if (t < tasks) quantize_task(st.a[i], st.b[i], t / groups >= Mr, t, xq);
    }
  }
  __syncthreads();

  // The consume step finds row r's bytes in its owner's region at
  // o_base + (owner's first row) * row_bytes, mod 4: o_base = (r0 * row_bytes) & 3,
  // the same for gate and up (weight pointers are dword aligned).
  global_f32* gy = (global_f32*)(yout);
  global_f32* gh = (global_f32*)(hout);
  const int o_base = static_cast<int>(reinterpret_cast<uintptr_t>(w + r0 * row_bytes) & 3u);
  stream_mt_consume<MT, TYPE, J, MODE>(chunk, off, o_base, rpw, r0, nrows, S, Mr, rows, region,
                                       sums_stride, gy, gh, xq, wlds, sums);
}

using StreamMtKernel = void (*)(StreamMtParams);

}  // namespace qk
