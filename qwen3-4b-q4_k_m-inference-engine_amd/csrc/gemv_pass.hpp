// Multi-pass whole-share mat-vec for one activation row: the M = 1 shapes
// whose per-CU share of the weights does not fit in LDS, chiefly the lm_head
// (151936 x 2560 Q6_K, 319 MB; src/Engine.cpp:106-111), optionally with the
// next-token argmax fused (src/cuda/argmax.cu:25-98).
//
// Replaces quantize + project<Q4_K/Q6_K> (src/cuda/matmul.cu:8-22, 86-125)
// for those shapes. The load discipline is the whole-share kernel's
// (gemv_stream.hpp): a wave reads contiguous byte runs of whole rows with
// 16-byte loads only (lane l takes bytes 16*(l + 64j) of the run), copies the
// chunks to its own LDS slot and reads the pieces from there. Here a wave's
// work is a sequence of passes of R whole rows each (R * row bytes <= J KB):
// a pass's chunks move from the registers to the wave's LDS slot, the next
// pass is issued into the same registers, and the pass is computed from LDS
// while the next one is in flight. Passes are dealt so that the whole
// GPU reads one contiguous window of the matrix at a time: pass p of worker k
// (k = workgroup * waves + wave, W workers) covers rows [(p*W + k)*R, +R) for
// p < full = N / (W*R); the rows left over (rest < W*R) are split evenly over
// the workers as one last pass of at most R rows.
//
// Per pass: rounds of 64 pieces (piece q: superblock q/4 of the pass, piece
// q%4), a quad's DPP sum per superblock into the wave's LDS sums, then a quad
// per row adds its row's superblock sums k, k+4, ... in order and the quad's
// DPP sum: the same pieces, order and arithmetic as the whole-share kernel,
// so results do not depend on timing. MODE 2 keeps each lane's best argmax
// key and ends with the device-wide candidate reduction of argmax.hpp.
#pragma once

#include "argmax.hpp"
#include "gemv_stream.hpp"

namespace qk {

constexpr int kPassWaves = 16;     // waves per workgroup (one workgroup per CU)
constexpr int kPassSums = 64;      // superblock sums per wave and pass, at most
constexpr int kPassMaxJ = 8;       // 16-byte loads per lane and pass, at most

struct PassParams {
  const float* x;          // [K]
  const uint8_t* w;        // [N rows x K], dword-aligned
  float* y;                // [N]; may be null in MODE 2
  void* argmax_ws;         // MODE 2: ArgmaxWorkspace
  uint32_t* argmax_result;  // MODE 2: index of the largest output
  int32_t K, S, N, R;      // R: rows per full pass
  int32_t full, rest, npass, pad;  // full rounds, rows of the last round, passes per worker
};

// Rows [ra, ra + nr) of pass `pass` of worker k of W.
struct PassRows {
  int64_t ra;
  int32_t nr;
};

__device__ __forceinline__ PassRows pass_rows(int pass, int k, int W, int R, int full, int N,
                                              int64_t last_a, int64_t last_b) {
  const bool in_full = pass < full;
  PassRows pr;
  pr.ra = in_full ? (static_cast<int64_t>(pass) * W + k) * R : last_a;
  pr.nr = in_full ? R : static_cast<int32_t>(last_b - last_a);
  return pr;
}

// A pass's run as 16-byte chunks from the dword boundary at or below its
// first byte (o bytes before it: Q6_K rows of an odd superblock count start
// 2-byte aligned): chunk c <= cmax covers run bytes [16c, 16c + 16), loaded
// through a buffer descriptor whose range ends at the dword boundary at or
// above the matrix end, so dwords past it read as zero and no byte outside the
// matrix's dwords is fetched.
struct PassRun {
  int64_t run4;  // byte offset of the run's first dword in the matrix
  int o, cmax;
};

__device__ __forceinline__ PassRun pass_run(int64_t row_bytes, PassRows pr) {
  const int64_t run = pr.ra * row_bytes;
  PassRun r;
  r.o = static_cast<int>(run & 3);  // w is dword-aligned
  r.run4 = run - r.o;
  r.cmax = max(static_cast<int>((r.o + pr.nr * row_bytes + 15) >> 4), 1) - 1;
  return r;
}

// Loads through the descriptor keep the weight stream out of the LDS wait
// counter (a flat load counts in both) and cost no per-lane address clamps.
template <int J>
__device__ __forceinline__ void pass_issue(u32x4 (&buf)[J], const PassRun& r, const uint8_t* w,
                                           int64_t end4, int lane) {
  constexpr int kNt = 2;  // cache policy: nontemporal (each byte is read once)
  const int64_t range = end4 - r.run4;
  const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(w) + r.run4, 0, static_cast<int>(min(range, int64_t{INT32_MAX})), 0x00020000);
#pragma unroll
  for (int j = 0; j < J; ++j)
    buf[j] = __builtin_amdgcn_raw_buffer_load_b128(rsrc, 16 * min(lane + 64 * j, r.cmax), 0, kNt);
}

template <int J>
__device__ __forceinline__ void pass_stage(const u32x4 (&buf)[J], const PassRun& r, lds_u8* slot,
                                           int lane) {
#pragma unroll
  for (int j = 0; j < J; ++j)
    *reinterpret_cast<lds_u32x4*>(slot + 16 * min(lane + 64 * j, r.cmax)) = buf[j];
}

// Pieces of the pass in rounds of 64, superblock sums, row totals.
template <int TYPE, int MODE>
__device__ __forceinline__ void pass_compute(PassRows pr, const PassRun& r, int S,
                                             const lds_u8* slot, const lds_q8_block* xq,
                                             lds_f32* sums, global_f32* y, uint64_t& key,
                                             int lane) {
  constexpr int B = TYPE == QK_TYPE_Q4_K ? kQ4KBytes : kQ6KBytes;
  const uint32_t pc = static_cast<uint32_t>(lane) & 3u;
  const int blk_a = piece_block_a(pc, TYPE), blk_step = piece_block_step(TYPE);
  const int npc = 4 * pr.nr * S;
  const int step = 16 % S;
  int s = (lane >> 2) % S;  // superblock within its row of the lane's piece, 16 superblocks a round
  for (int q0 = 0; q0 < npc; q0 += 64) {
    const int q = q0 + lane;
    const int sbw = min(q, npc - 1) >> 2;  // lanes past the pass redo its last superblock, store nothing
    const lds_u8* sbp = slot + r.o + __umul24(sbw, B);  // full-rate multiply (sbw < 2^24)
    const lds_q8_block* xr = xq + ((s * 8 + blk_a) & 0xFFFF);
    float v;
    if constexpr (TYPE == QK_TYPE_Q4_K)
      v = dot_q4k_piece(lds_q4k_piece(sbp, pc), load_x(xr), load_x(xr + blk_step), pc);
    else
      v = dot_q6k_piece(lds_q6k_piece(sbp, pc), load_x(xr), load_x(xr + blk_step), pc);
    v = add_dpp<0xB1>(v);
    v = add_dpp<0x4E>(v);
    if (pc == 0 && q < npc) sums[sbw] = v;
    s += step;
    if (s >= S) s -= S;
  }
  asm volatile("" ::: "memory");  // the wave's reads below follow its writes
  // a quad per row: lane k adds the row's sums k, k+4, ... in order
  const int i = lane >> 2;
  if (i < pr.nr) {
    float t = 0.0f;
    for (int c = static_cast<int>(pc); c < S; c += 4) t += sums[i * S + c];
    t = add_dpp<0x4E>(add_dpp<0xB1>(t));
    if (pc == 0) {
      const int64_t row = pr.ra + i;
      if (MODE == 0 || y != nullptr) y[row] = t;
      if constexpr (MODE == 2) key = max_key(key, argmax_key(t, static_cast<uint32_t>(row)));
    }
  }
  asm volatile("" ::: "memory");  // the next pass's sums follow these reads
}

// MODE 0: y = x . W^T; MODE 2: the same (y optional) and *argmax_result =
// argmax of y by the reference's rules. kPassWaves waves per workgroup, one
// workgroup per CU. One register buffer per wave: while a pass is computed
// from the wave's LDS slot, the next pass is in flight into the registers.
// (Measured on the lm_head: 16 waves with one buffer 57.8 us; 8 or 12 waves
// with two buffers 59-62 us; the two-buffer 16-wave form exceeds 128 VGPRs.)
template <int TYPE, int MODE, int J>
__global__ __launch_bounds__(64 * kPassWaves) void pass_matvec_kernel(const PassParams p) {
  extern __shared__ __align__(16) unsigned char lds_raw[];
  __shared__ uint64_t keys[kPassWaves + 1];
  constexpr int B = TYPE == QK_TYPE_Q4_K ? kQ4KBytes : kQ6KBytes;
  // Every argument in one scalar-load round (see matvec_kernel).
  asm volatile("" ::"s"(p.x), "s"(p.w), "s"(p.y), "s"(p.argmax_ws), "s"(p.argmax_result), "s"(p.K),
               "s"(p.S), "s"(p.N), "s"(p.R), "s"(p.full), "s"(p.rest), "s"(p.npass), "s"(p.pad));
  __builtin_amdgcn_sched_barrier(0);
  const int K = p.K;
  const int lane = static_cast<int>(threadIdx.x & 63u);
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));

  // The activation loads of the quantiser waves go out first.
  const int nq = min(kPassWaves, (K / 8 + 64 * kXStaged - 1) / (64 * kXStaged));
  XStage<1> stage;
  if (wave < nq) stage_x<1>(p.x, 1, K, nq, stage);
  __builtin_amdgcn_sched_barrier(0);

  int S = p.S, N = p.N, R = p.R, full = p.full, npass = p.npass;
  const int W = static_cast<int>(gridDim.x) * kPassWaves;
  const int k = static_cast<int>(blockIdx.x) * kPassWaves + wave;
  const int64_t base = static_cast<int64_t>(full) * W * R;
  int64_t last_a = base + static_cast<int64_t>(k) * p.rest / W;
  int64_t last_b = base + static_cast<int64_t>(k + 1) * p.rest / W;
  const uint8_t* w = p.w;
  global_f32* y = (global_f32*)(p.y);
  // Values used after the barrier are held in registers: left as kernel
  // arguments, the compiler re-reads them from memory there.
  asm volatile("" : "+s"(S), "+s"(N), "+s"(R), "+s"(full), "+s"(npass), "+s"(last_a), "+s"(last_b),
               "+s"(w), "+s"(y));
  const int64_t row_bytes = static_cast<int64_t>(S) * B;
  // the dword boundary at or above the matrix end (w is dword-aligned)
  const int64_t end4 = (static_cast<int64_t>(N) * row_bytes + 3) & ~int64_t{3};

  u32x4 buf[J];
  PassRows pr = pass_rows(0, k, W, R, full, N, last_a, last_b);
  PassRun run = pass_run(row_bytes, pr);
  pass_issue<J>(buf, run, w, end4, lane);
  __builtin_amdgcn_sched_barrier(0);

  lds_q8_block* xq = (lds_q8_block*)(lds_raw);
  lds_u8* slot = (lds_u8*)(lds_raw) + S * 8 * static_cast<int>(sizeof(qk_q8_block)) + wave * (J * 1024);
  lds_f32* sums = reinterpret_cast<lds_f32*>((lds_u8*)(lds_raw) + S * 8 * static_cast<int>(sizeof(qk_q8_block)) +
                                             kPassWaves * J * 1024) + wave * kPassSums;
  if (wave < nq) quantize_staged_into_lds<1>(1, K, nq, stage, xq);  // K <= kStreamMaxK: all staged
  __syncthreads();

  uint64_t key = 0;
  // The issue is unconditional (a load under a branch makes the compiler
  // wait for every load at the join); the last pass is peeled.
  for (int pass = 0; pass + 1 < npass; ++pass) {
    pass_stage<J>(buf, run, slot, lane);
    const PassRows pr2 = pass_rows(pass + 1, k, W, R, full, N, last_a, last_b);
    const PassRun run2 = pass_run(row_bytes, pr2);
    pass_issue<J>(buf, run2, w, end4, lane);
    pass_compute<TYPE, MODE>(pr, run, S, slot, xq, sums, y, key, lane);
    pr = pr2;
    run = run2;
  }
  pass_stage<J>(buf, run, slot, lane);
  pass_compute<TYPE, MODE>(pr, run, S, slot, xq, sums, y, key, lane);
  if constexpr (MODE == 2)
    argmax_finish(key, static_cast<ArgmaxWorkspace*>(p.argmax_ws), p.argmax_result, keys, kPassWaves);
}

using PassKernel = void (*)(PassParams);

}  // namespace qk
