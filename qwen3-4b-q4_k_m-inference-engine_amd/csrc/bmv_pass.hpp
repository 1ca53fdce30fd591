// Multi-pass batched mat-vec on the int8 matrix cores: M = 2..8 activation
// rows against a very tall matrix (the lm_head, 151936 x 2560 Q6_K:
// src/Engine.cpp:106-111 with a batch of sequences). Replaces quantize +
// project<Q4_K/Q6_K> with gridDim.y = rows (src/cuda/matmul.cu:8-22, 86-125,
// 151-158) for those shapes.
//
// The tile arithmetic is the batched kernels' (bmv.hpp: one
// v_mfma_i32_16x16x64_i8 takes 16 weight rows against a block-diagonal
// activation tile, the sub-block and Q8 scales applied in fp32 per tile);
// the load discipline is the multi-pass kernel's (gemv_pass.hpp): each wave
// streams its own work through its own LDS slot with 16-byte loads only, one
// pass in flight in registers while the previous one is computed from LDS,
// and no workgroup barrier after the activation quantisation.
//
// Work: 16-row groups of the matrix, dealt round-robin to the waves of the
// launch (group g to wave g % W), so at any moment the GPU streams one
// compact window of the matrix. A pass is one group's 16 rows x C superblock
// columns [c0, c0 + C): 16 runs of C * B bytes (one per row), each read from
// the dword boundary at or below its first byte in `cpr` 16-byte chunks;
// run r lands at slot + 16 * cpr * r. Lane (n, kq) then takes its row n's
// superblocks of the pass from the slot as the whole-share batched kernel
// does (bmv_ws.hpp: ws_tile), accumulates the group's tiles over its
// ceil(S / C) passes in registers, and after the group's last pass the lanes
// of a row add their partial sums and store the row's M outputs.
#pragma once

#include "bmv_ws.hpp"

namespace qk {

constexpr int kBpWaves = 8;     // waves per workgroup (one workgroup per CU)
constexpr int kBpXStaged = 5;   // fp32 activation tasks per thread staged ahead of the weights
constexpr int kBpMaxJ = 8;      // 16-byte chunks per lane and pass, at most

struct BmvPassParams {
  const float* x;    // [M x K]
  const uint8_t* w;  // [N rows x K], dword-aligned
  float* y;          // [M x N]
  int32_t M, K, S, N;
  int32_t stride;    // LDS bytes per activation row of codes (K + 16)
  int32_t act;       // LDS bytes of the activation image (16-byte multiple)
  int32_t C, cpr;    // superblock columns per pass, chunks per run
  int32_t ppg, pad;  // passes per group (ceil(S / C))
};

// Rows of one pass: group g (rows 16g .. 16g + 15, clamped to N - 1: rows
// past the matrix re-read its last row and are never stored), columns
// [c0, c0 + C) (clamped to S: a short last pass re-reads the last column,
// never computed).
template <int TYPE, int J>
__device__ __forceinline__ void bp_issue(u32x4 (&buf)[J], const BmvPassParams& p, __amdgpu_buffer_rsrc_t rsrc,
                                         int g, int c0, const int (&run)[J], const int (&q)[J]) {
  constexpr int B = TYPE == QK_TYPE_Q4_K ? kQ4KBytes : kQ6KBytes;
  // Cache policy: default. A run of C superblocks starts and ends inside
  // 128-byte lines that the row's neighbouring passes (the same wave's next
  // ones) also read; with the nontemporal hint those lines left the L2 in
  // between and were fetched again: FETCH_SIZE 1.26x the matrix at M = 8,
  // 1.03x without the hint (lm_head 97-105 -> 94-98 us).
  constexpr int kNt = 0;
  const int64_t row_bytes = static_cast<int64_t>(p.S) * B;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int64_t row = min(16 * g + run[j], p.N - 1);
    const int64_t first = row * row_bytes + static_cast<int64_t>(min(c0, p.S - 1)) * B;
    buf[j] = __builtin_amdgcn_raw_buffer_load_b128(rsrc, static_cast<int>((first & ~int64_t{3}) + 16 * q[j]), 0, kNt);
  }
}

template <int TYPE, int J>
__global__ __launch_bounds__(64 * kBpWaves) void bmv_pass_kernel(const BmvPassParams p) {
  extern __shared__ __align__(16) unsigned char lds_raw[];
  constexpr int B = TYPE == QK_TYPE_Q4_K ? kQ4KBytes : kQ6KBytes;
  asm volatile("" ::"s"(p.x), "s"(p.w), "s"(p.y), "s"(p.M), "s"(p.K), "s"(p.S), "s"(p.N), "s"(p.stride),
               "s"(p.act), "s"(p.C), "s"(p.cpr), "s"(p.ppg), "s"(p.pad));
  __builtin_amdgcn_sched_barrier(0);
  const int K = p.K, M = p.M, S = p.S, N = p.N, stride = p.stride;
  const int C = p.C, cpr = p.cpr, ppg = p.ppg;
  const int tid = static_cast<int>(threadIdx.x);
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  // activations first: fp32 tasks of 8 values, the first kBpXStaged per
  // thread loaded ahead of the weights
  const int groups8 = K / 8, tasks = M * groups8;
  f32x4 xa[kBpXStaged], xb[kBpXStaged];
#pragma unroll
  for (int i = 0; i < kBpXStaged; ++i)
    load_x_group(p.x, M, K, min(tid + 64 * kBpWaves * i, tasks - 1), xa[i], xb[i]);
  __builtin_amdgcn_sched_barrier(0);

  // this wave's passes: groups wid, wid + W, ...; pass i = group i / ppg,
  // columns from (i % ppg) * C
  const int W = static_cast<int>(gridDim.x) * kBpWaves;
  const int wid = wave * static_cast<int>(gridDim.x) + static_cast<int>(blockIdx.x);
  const int groups = (N + 15) / 16;
  const int ngroups = wid < groups ? (groups - 1 - wid) / W + 1 : 0;
  const int npass = ngroups * ppg;
  // each lane's chunks of a pass: chunk c = lane + 64 j (clamped to the last)
  // of run c / cpr, chunk c % cpr of the run
  const int nchunks = 16 * cpr;
  int run[J], q[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int c = min(lane + 64 * j, nchunks - 1);
    run[j] = c / cpr;
    q[j] = c - run[j] * cpr;
  }
  // loads through a descriptor whose range ends at the dword boundary at or
  // above the matrix end: dwords past it read as zero
  const int64_t end4 = (static_cast<int64_t>(N) * S * B + 3) & ~int64_t{3};
  const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(p.w), 0, static_cast<int>(min(end4, int64_t{INT32_MAX})), 0x00020000);
  auto pass_at = [&](int i, int& g, int& c0) {
    const int gi = i / ppg;
    g = wid + W * gi;
    c0 = (i - gi * ppg) * C;
  };
  u32x4 buf[J];
  {
    int g, c0;
    pass_at(0, g, c0);
    bp_issue<TYPE, J>(buf, p, rsrc, min(g, groups - 1), c0, run, q);
  }
  __builtin_amdgcn_sched_barrier(0);

  lds_u8* codes = (lds_u8*)(lds_raw);
  lds_f32* xs = (lds_f32*)(lds_raw + bmv_lds_z(stride));
  lds_f32* xss = xs + K / 4;
  lds_f32* xf = xs + K / 2;
  lds_u8* slot = (lds_u8*)(lds_raw + p.act) + wave * (J * 1024);
#pragma unroll
  for (int i = 0; i < kBpXStaged; ++i) {
    const int t = tid + 64 * kBpWaves * i;
    if (t < tasks) bmv_quantize_task(xa[i], xb[i], t, groups8, stride, codes, xs, xss, xf);
  }
  for (int t = tid + 64 * kBpWaves * kBpXStaged; t < tasks; t += 64 * kBpWaves) {
    f32x4 a, b;
    load_x_group(p.x, M, K, t, a, b);
    bmv_quantize_task(a, b, t, groups8, stride, codes, xs, xss, xf);
  }
  if (tid == 0) *reinterpret_cast<lds_u32x4*>(codes + 8 * stride) = u32x4{0u, 0u, 0u, 0u};
  __syncthreads();

  BmvLane L;
  L.n = lane & 15;
  L.kq = lane >> 4;
  L.zero = static_cast<uint32_t>(8 * stride);
  L.a4_valid = (L.n < 8) == (L.kq < 2);
  L.a4_base = static_cast<uint32_t>((L.n & 7) * stride + 16 * (L.kq & 1));
  L.a6_valid = (L.n >> 2) == L.kq;
  L.a6_base = static_cast<uint32_t>((L.n & 3) * stride + 16 * L.kq);
  const int64_t row_bytes = static_cast<int64_t>(S) * B;
  const lds_u8* my_run = slot + 16 * cpr * L.n;  // lane's row's run

  auto body = [&](auto mh) {
    constexpr int MH = decltype(mh)::value;
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
    for (int i = 0; i < npass; ++i) {
      int g, c0;
      pass_at(i, g, c0);
      // the pass's chunks into the slot (the previous pass's reads of it
      // came first in this wave's program order)
#pragma unroll
      for (int j = 0; j < J; ++j)
        *reinterpret_cast<lds_u32x4*>(slot + 16 * (run[j] * cpr + q[j])) = buf[j];
      asm volatile("" ::: "memory");
      {  // the next pass (the last one again past the end), unconditionally
        int g2, c2;
        pass_at(min(i + 1, npass - 1), g2, c2);
        bp_issue<TYPE, J>(buf, p, rsrc, g2, c2, run, q);
      }
      // this lane's row of the group and where its run starts in the slot
      const int row = min(16 * g + L.n, N - 1);
      const uint32_t o = static_cast<uint32_t>((row * row_bytes + static_cast<int64_t>(c0) * B) & 3);
#pragma unroll 1
      for (int cc = 0; cc < C; ++cc) {
        const int s = c0 + cc;
        if (s < S) {
          if constexpr (TYPE == QK_TYPE_Q4_K) {
            Q4Tile t;
            ws_tile(t, my_run + o + cc * B, L.kq);
            bmv_tile(t, s, L, stride, codes, xs, xss, acc);
          } else {
            Q6Tile t;
            ws_tile(t, my_run + o + cc * B, L.kq);
            bmv_tile<MH>(t, s, L, stride, codes, xs, xf, acc);
          }
        }
      }
      asm volatile("" ::: "memory");  // the next pass's slot writes follow these reads
      if (c0 + C >= S) {  // the group's last pass: row totals of the lanes, store
        const int r = 16 * g + L.n;
        if constexpr (TYPE == QK_TYPE_Q4_K) {
          f32x4 v;
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = swap32_sum(acc[e]);  // both sub-block sets
          if (L.kq < 2 && r < N) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int m = 4 * L.kq + e;
              if (m < M) p.y[static_cast<int64_t>(m) * N + r] = v[e];
            }
          }
        } else {
          f32x4 v[2];
#pragma unroll
          for (int h = 0; h < MH; ++h)
#pragma unroll
            for (int e = 0; e < 4; ++e) v[h][e] = swap16_sum(swap32_sum(acc[h][e]));  // all four kq
          if (L.kq == 0 && r < N) {
#pragma unroll
            for (int h = 0; h < MH; ++h)
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                const int m = 4 * h + e;
                if (m < M) p.y[static_cast<int64_t>(m) * N + r] = v[h][e];
              }
          }
        }
        clear();
      }
    }
  };
  if (TYPE == QK_TYPE_Q4_K || M <= 4)
    body(std::integral_constant<int, 1>{});
  else
    body(std::integral_constant<int, 2>{});
}

using BmvPassKernel = void (*)(BmvPassParams);

}  // namespace qk
