// Whole-share mat-vec for one activation row (M = 1 decode projections whose
// per-CU share of the weights fits in LDS).
//
// Replaces quantize + project<Q4_K/Q6_K> (src/cuda/matmul.cu:8-22, 86-125)
// for the decode shapes (src/Engine.cpp:83-109). The issue rate of vector
// memory instructions bounds a one-burst launch on gfx950: every wave64 load
// costs the CU's texture addresser the same ~16 cycles whatever its width, so
// the per-piece layout of the streaming kernel (3 loads per Q4_K piece, with
// the 16-byte header read by all 4 lanes of a superblock; 9 per Q6_K piece,
// five of them 2- or 4-byte) spends 2.3-4x the instructions of a plain read.
// Here each workgroup owns a contiguous range of rows and each wave a
// contiguous run of whole superblocks of it, which the wave reads with
// 16-byte loads only (lane l takes bytes 16*(l + 64j) of the run), all issued
// at once before the activation quantisation. The chunks are then copied to
// the wave's own LDS region, from which its lanes read the pieces (header
// broadcasts and the Q6_K realignment cost LDS reads, not memory
// instructions). Per-superblock sums go to LDS; after one barrier each row's
// sums are added in a fixed order and stored, so results do not depend on
// timing.
#pragma once

#include "gemv_kernel.hpp"

namespace qk {

constexpr int kStreamWaves = 16;  // waves per workgroup (one workgroup per CU)
constexpr int kStreamMaxJ = 8;    // 16-byte loads per lane, at most
// Widest activation row: every quantiser lane's tasks are staged ahead of the weights.
constexpr int kStreamMaxK = 8 * 64 * kStreamWaves * kXStaged;

// One weight matrix of a whole-share launch. Workgroup wg_begin + g takes
// rows [g*per + min(g, rem), (g+1)*per + min(g+1, rem)) with per = rows /
// wg_count and rem = rows % wg_count (no division in the kernel).
struct StreamSegment {
  const uint8_t* w;
  float* y;
  int32_t rows;
  int32_t type;
  int32_t wg_begin;
  int32_t per;
  int32_t rem;
  int32_t pad;
};

// mode 0: y_j = x . W_j^T for every segment; mode 1: seg[0] = gate and
// seg[1] = up over the same workgroups, h = SiLU(x . gate^T) * (x . up^T).
struct StreamParams {
  const float* x;
  float* h;
  int32_t K, S, nseg, max_sb;  // max_sb: superblocks of the largest workgroup share (per part)
  StreamSegment seg[kMaxSegments];
  const float* norm;  // MODE 3: RMSNorm scale [K]
  float eps;          // MODE 3: RMSNorm epsilon
  int32_t pad;
};

typedef __attribute__((address_space(3))) uint8_t lds_u8;
typedef __attribute__((address_space(3))) uint32_t lds_u32;
typedef __attribute__((address_space(3))) uint16_t lds_u16;
typedef __attribute__((address_space(3))) float lds_f32;
typedef __attribute__((address_space(1))) float global_f32;

__device__ __forceinline__ uint32_t lds_offset(const lds_u8* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p));
}

// Pieces read from a superblock in LDS (same register images as the global
// loads of the streaming kernel). Q4_K superblocks sit at 16-byte aligned
// offsets; Q6_K ones at 2-byte aligned offsets, read as dwords from the
// boundary below and realigned by the dot (Q6KPiece::shift).
__device__ __forceinline__ Q4KPiece lds_q4k_piece(const lds_u8* sb, uint32_t j) {
  const lds_u32x4* v = reinterpret_cast<const lds_u32x4*>(sb);
  Q4KPiece f;
  f.head = v[0];
  f.q0 = v[1 + 2 * j];
  f.q1 = v[2 + 2 * j];
  return f;
}

__device__ __forceinline__ Q6KPiece lds_q6k_piece(const lds_u8* sb, uint32_t p) {
  const uint32_t h = p >> 1, r = p & 1u;
  const uint32_t mis = lds_offset(sb) & 3u;  // 0 or 2
  const lds_u32* base = reinterpret_cast<const lds_u32*>(sb - mis);
  const lds_u32* ql = base + 16 * h + 8 * r;
  const lds_u32* qh = base + 32 + 8 * h;
  Q6KPiece f;
  f.l0 = u32x4{ql[0], ql[1], ql[2], ql[3]};
  f.l1 = u32x4{ql[4], ql[5], ql[6], ql[7]};
  f.l2 = ql[8];
  f.h0 = u32x4{qh[0], qh[1], qh[2], qh[3]};
  f.h1 = u32x4{qh[4], qh[5], qh[6], qh[7]};
  f.h2 = qh[8];
  const lds_u16* sc = reinterpret_cast<const lds_u16*>(sb + 192 + 8 * h + 2 * r);
  f.sc_a = sc[0];
  f.sc_b = sc[2];
  f.d_bits = *reinterpret_cast<const lds_u16*>(sb + 208);
  f.shift = 8 * mis;
  return f;
}

// A wave's share: superblocks [sb_a, sb_b) of its part (MODE 1: waves 0-7
// gate, 8-15 up) of the workgroup's rows, held as 16-byte chunks: lane l's
// chunk j covers run bytes [off(j), off(j) + 16) from the dword boundary at or
// below the run start (o bytes before it; Q4_K runs are 16-byte aligned).
// off(j) = 16 * min(l + 64 j, cmax), or lim for a chunk moved back to end at
// the matrix's last dword boundary (recomputed where it is used rather than
// held in J registers).
template <int J>
struct WaveShare {
  u32x4 chunk[J];
  int cmax, lim;
  int sb_a, sb_b, o, part;
  __device__ __forceinline__ int off(int j, int lane) const {
    return min(16 * min(lane + 64 * j, cmax), lim);
  }
};

// Issues the 16-byte loads of a wave's share: superblocks [sb_a, sb_b) of
// rows [r0, ...) of a matrix of `rows` rows of S superblocks of B bytes at w
// (dword-aligned). An empty share reads the run's first chunk. The matrix's
// last chunk is moved back so it ends at the dword boundary at or above the
// matrix end: no byte outside the matrix's dwords is read. (Addresses stay
// pointer arithmetic on the kernel argument, so the compiler keeps them in
// the global address space: global loads, whose waits count in order.)
// J0, J1: only chunks [J0, J1) are loaded (a share issued in two parts; both
// calls take the same share arguments).
template <int J, int J0 = 0, int J1 = J>
__device__ __forceinline__ void issue_share(WaveShare<J>& ws, const uint8_t* w, int rows, int r0,
                                            int S, int B, int lane) {
  static_assert(0 <= J0 && J0 < J1 && J1 <= J, "chunk range");
  const int64_t row_bytes = static_cast<int64_t>(S) * B;
  const uint8_t* run = w + r0 * row_bytes + static_cast<int64_t>(ws.sb_b > ws.sb_a ? ws.sb_a : 0) * B;
  ws.o = static_cast<int>(reinterpret_cast<uintptr_t>(run) & 3u);  // 0 or 2 (Q6_K), 0 (Q4_K)
  const uint8_t* run4 = run - ws.o;
  ws.cmax = max((ws.o + (ws.sb_b - ws.sb_a) * B + 15) >> 4, 1) - 1;
  // w is dword-aligned: the last dword boundary at or above the matrix end
  const uint8_t* last = w + ((rows * row_bytes + 3) & ~int64_t{3}) - 16;
  ws.lim = static_cast<int>(last - run4);
#pragma unroll
  for (int jj = J0; jj < J1; ++jj) {
    const uint8_t* a = run4 + 16 * min(lane + 64 * jj, ws.cmax);
    a = a < last ? a : last;
    ws.chunk[jj] = stream_load16_a4(a);
  }
}

// Consumes the share after the activation barrier: chunks into the wave's
// LDS region as they arrive (the waits count the loads issued after each
// one), rounds of 64 pieces from there (piece q of the run: superblock q/4,
// piece q%4), superblock sums to LDS, a barrier, then the row totals. Only a
// chunk moved back at the matrix end can sit off a 16-byte boundary.
// IL: each round right after the chunks it needs (measured faster for the
// mixed-type q/k/v launch and the fused FFN's gate/up phase); otherwise every
// chunk first, then the rounds.
// SCALED: row totals are multiplied by out_scale (the RMSNorm fold).
// AGENT_H: h is stored with agent-scope coherent stores (read back by other
// workgroups of the same launch, the fused FFN). ROW_WAVE0, ROW_WAVES: the
// waves that form the row totals. HOOK_AT: when >= 0, hook() runs right after
// chunk HOOK_AT is in LDS, before the rounds that chunk completes (the fused
// FFN issues its next loads there, once its share has arrived).
// A row's total from its S superblock sums by one lane, in the order of a
// quad's (lane k adds sums k, k+4, ... in order from 0; then the DPP sums
// (s0 + s1) + (s2 + s3)), so both give the same bits.
__device__ __forceinline__ float row_total_one_lane(const lds_f32* r, int S) {
  float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
  int t = 0;
  for (; t + 4 <= S; t += 4) {
    s0 += r[t];
    s1 += r[t + 1];
    s2 += r[t + 2];
    s3 += r[t + 3];
  }
  if (t < S) s0 += r[t];
  if (t + 1 < S) s1 += r[t + 1];
  if (t + 2 < S) s2 += r[t + 2];
  return (s0 + s1) + (s2 + s3);
}

struct NoHook {
  __device__ __forceinline__ void operator()() const {}
};
template <int TYPE, int J, int MODE, bool IL, bool SCALED = false, bool AGENT_H = false,
          int ROW_WAVE0 = 0, int ROW_WAVES = kStreamWaves, int HOOK_AT = -1, typename Hook = NoHook>
__device__ __forceinline__ void stream_consume(const WaveShare<J>& ws, int S, int max_sb, int r0,
                                               int r1, global_f32* yout, global_f32* hout,
                                               const lds_q8_block* xq, lds_u8* wlds,
                                               lds_f32* sums, float out_scale, Hook hook = Hook{}) {
  constexpr int B = TYPE == QK_TYPE_Q4_K ? kQ4KBytes : kQ6KBytes;
  const int lane = static_cast<int>(threadIdx.x & 63u);
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int sb_a = ws.sb_a, sb_b = ws.sb_b, o = ws.o;
  lds_u8* reg = wlds + wave * (J * 1024);
  const int npc = 4 * (sb_b - sb_a);
  const int rounds = (npc + 63) >> 6;
  const uint32_t pc = static_cast<uint32_t>(lane) & 3u;
  const int blk_a = piece_block_a(pc, TYPE), blk_step = piece_block_step(TYPE);
  // s = superblock within its row of the lane's superblock in the current
  // round, stepped by 16 superblocks per round
  const int step = 16 % S;
  int s = (sb_a + (lane >> 2)) % S;
  auto round_chunks = [&](int r) { return (o + min(16 * (r + 1), sb_b - sb_a) * B + 15) >> 4; };
  auto compute = [&](int r) {
    const int q = 64 * r + lane;
    const int sbw = min(q, npc - 1) >> 2;  // lanes past the run redo the last superblock, store nothing
    const lds_u8* sbp = reg + o + __umul24(sbw, B);  // full-rate multiply (sbw < 2^24)
    const lds_q8_block* xr = xq + ((s * 8 + blk_a) & 0xFFFF);
    float v;
    if constexpr (TYPE == QK_TYPE_Q4_K)
      v = dot_q4k_piece(lds_q4k_piece(sbp, pc), load_x(xr), load_x(xr + blk_step), pc);
    else
      v = dot_q6k_piece(lds_q6k_piece(sbp, pc), load_x(xr), load_x(xr + blk_step), pc);
    v = add_dpp<0xB1>(v);
    v = add_dpp<0x4E>(v);
    if (pc == 0 && q < npc) sums[ws.part * max_sb + sb_a + sbw] = v;
    s += step;
    if (s >= S) s -= S;
  };
  auto write_chunk = [&](int j) {
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
  };
  if constexpr (IL) {
    int r = 0;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      write_chunk(j);
      if (j == HOOK_AT) {
        __builtin_amdgcn_sched_barrier(0);  // the hook's loads stay after this chunk's wait
        hook();
        __builtin_amdgcn_sched_barrier(0);
      }
      asm volatile("" ::: "memory");  // the wave's reads below follow its writes
      for (; r < rounds && round_chunks(r) <= 64 * (j + 1); ++r) compute(r);
    }
  } else {
#pragma unroll
    for (int j = 0; j < J; ++j) {
      write_chunk(j);
      if (j == HOOK_AT) {
        __builtin_amdgcn_sched_barrier(0);  // the hook's loads stay after this chunk's wait
        hook();
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    asm volatile("" ::: "memory");  // the wave's reads below follow its writes
    for (int r = 0; r < rounds; ++r) compute(r);
  }
  __syncthreads();

  // Row totals, a quad per row: lane k of the quad adds the row's superblock
  // sums k, k+4, ... in order, then the quad's DPP sum.
  const int nrows = r1 - r0;
  const int rt = static_cast<int>(threadIdx.x) - 64 * ROW_WAVE0;
  // When only some waves form the totals (the fused FFN, whose other waves go
  // on to VALU-heavy work on the same SIMDs), they run at raised priority
  // (sharing the SIMD evenly made one wave's 38 totals take ~2.5 us), one lane
  // per row, adding the row's sums in the quad order below.
  constexpr bool kPrio = ROW_WAVES < kStreamWaves;
  const int k = kPrio ? 0 : lane & 3;
  const int first = rt >= 0 && rt < 64 * ROW_WAVES ? (kPrio ? rt : rt >> 2) : nrows;
  if constexpr (kPrio) {
    if (first < nrows) __builtin_amdgcn_s_setprio(3);
  }
  for (int i = first; i < nrows; i += (kPrio ? 64 : 16) * ROW_WAVES) {
    float g, u = 0.0f;
    if constexpr (kPrio) {
      g = row_total_one_lane(sums + i * S, S);
      if constexpr (MODE == 1) u = row_total_one_lane(sums + max_sb + i * S, S);
    } else {
      g = 0.0f;
      for (int t = k; t < S; t += 4) {
        g += sums[i * S + t];
        if constexpr (MODE == 1) u += sums[max_sb + i * S + t];
      }
      g = add_dpp<0x4E>(add_dpp<0xB1>(g));
      if constexpr (MODE == 1) u = add_dpp<0x4E>(add_dpp<0xB1>(u));
    }
    if constexpr (SCALED) {
      g *= out_scale;
      u *= out_scale;
    }
    if (k == 0) {
      if constexpr (MODE == 0) {
        yout[r0 + i] = g;
      } else {
        const float hv = (g / (1.0f + expf(-g))) * u;
        if constexpr (AGENT_H)
          __hip_atomic_store(hout + r0 + i, hv, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        else
          hout[r0 + i] = hv;
      }
    }
  }
  if constexpr (kPrio) __builtin_amdgcn_s_setprio(0);
}

// TYPE: the weight type of every segment, or 0 for segments of both types.
// Everything up to the activation barrier is type-independent (the bytes per
// superblock are a runtime value), so the loads of both types are issued by
// the same straight-line code and the quantiser's waits count them exactly;
// only the consumption is specialised per type.
// MODE 0: y_j = x . W_j^T per segment; 1: h = SiLU(x . gate^T) * (x . up^T);
// 3: mode 1 on RMSNorm(x) = (x * inv) * scale, inv = rsqrt(mean(x^2) + eps)
// (src/cuda/rms_norm.cu:6-24 folded into the launch). The Q8 round trip is
// scale-invariant (codes = round(127 v / amax), block scale amax / 127), so
// the quantiser waves quantise x * scale as soon as their activations arrive,
// with no wait for the row's sum of squares, and the gate and up row totals
// are multiplied by inv instead; the sum's wave partials go to LDS before the
// activation barrier. Against quantising the normalised row this moves
// only fp32 rounding (a code can step at a near-tie), while |x * scale| stays
// in fp32's normal range.
template <int TYPE, int J, int MODE>
__global__ __launch_bounds__(64 * kStreamWaves) void stream_matvec_kernel(const StreamParams p) {
  extern __shared__ __align__(16) unsigned char lds_raw[];
  constexpr bool kFfn = MODE == 1 || MODE == 3;
  constexpr int kParts = kFfn ? 2 : 1;
  constexpr int kWpp = kStreamWaves / kParts;  // waves per part
  // Every argument in one scalar-load round (see matvec_kernel).
#pragma unroll
  for (int j = 0; j < kMaxSegments; ++j)
    asm volatile("" ::"s"(p.seg[j].w), "s"(p.seg[j].y), "s"(p.seg[j].rows), "s"(p.seg[j].type),
                 "s"(p.seg[j].wg_begin), "s"(p.seg[j].per), "s"(p.seg[j].rem), "s"(p.seg[j].pad));
  asm volatile("" ::"s"(p.x), "s"(p.h), "s"(p.K), "s"(p.S), "s"(p.nseg), "s"(p.max_sb));
  if constexpr (MODE == 3) asm volatile("" ::"s"(p.norm), "s"(p.eps));
  __builtin_amdgcn_sched_barrier(0);
  const int K = p.K, nseg = p.nseg;

  // The activation loads of the quantiser waves go out first.
  // (capped by this kernel's own wave count: K <= kStreamMaxK stages every task)
  const int nq = min(kStreamWaves, (K / 8 + 64 * kXStaged - 1) / (64 * kXStaged));
  const int lane = static_cast<int>(threadIdx.x & 63u);
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  XStage<1> stage, nstage;  // nstage: MODE 3's norm scale of the staged tasks
  if (wave < nq) {
    stage_x<1>(p.x, 1, K, nq, stage);
    if constexpr (MODE == 3) stage_x<1>(p.norm, 1, K, nq, nstage);
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
  const int rows = pick(p.seg[0].rows, p.seg[1].rows, p.seg[2].rows, p.seg[3].rows);
  const int type = TYPE != 0 ? TYPE : pick(p.seg[0].type, p.seg[1].type, p.seg[2].type, p.seg[3].type);
  const int g = wg - pick(p.seg[0].wg_begin, p.seg[1].wg_begin, p.seg[2].wg_begin, p.seg[3].wg_begin);
  const int per = pick(p.seg[0].per, p.seg[1].per, p.seg[2].per, p.seg[3].per);
  const int rem = pick(p.seg[0].rem, p.seg[1].rem, p.seg[2].rem, p.seg[3].rem);
  int r0 = g * per + min(g, rem);
  int r1 = r0 + per + (g < rem ? 1 : 0);
  // Values used after the barriers are held in registers: left as kernel
  // arguments, the compiler re-reads them from memory there (a round trip).
  int S = p.S, max_sb = p.max_sb;
  float* hout = p.h;
  asm volatile("" : "+s"(S), "+s"(max_sb), "+s"(hout), "+s"(yout), "+s"(r0), "+s"(r1));
  float eps = 0.0f;
  if constexpr (MODE == 3) {
    eps = p.eps;
    asm volatile("" : "+s"(eps));
  }

  // The wave's run [sb_a, sb_b) as 16-byte chunks (an idle wave reads the
  // workgroup's first chunk).
  const int B = type == QK_TYPE_Q4_K ? kQ4KBytes : kQ6KBytes;
  WaveShare<J> ws;
  ws.part = wave / kWpp;
  const int wv = wave % kWpp;
  const int nsb = (r1 - r0) * S;  // superblocks of the workgroup, per part
  ws.sb_a = nsb * wv / kWpp;
  ws.sb_b = nsb * (wv + 1) / kWpp;
  issue_share<J>(ws, kFfn && ws.part ? p.seg[1].w : w0, rows, r0, S, B, lane);
  __builtin_amdgcn_sched_barrier(0);

  lds_q8_block* xq = (lds_q8_block*)(lds_raw);
  lds_u8* wlds = (lds_u8*)(lds_raw) + S * 8 * static_cast<int>(sizeof(qk_q8_block));
  lds_f32* sums = reinterpret_cast<lds_f32*>(wlds + kStreamWaves * J * 1024);
  // MODE 3: the quantiser waves' partial sums of squares, after the
  // superblock sums of both parts
  lds_f32* norm_part = sums + 2 * max_sb;
  if constexpr (MODE == 3) {
    if (wave < nq) {
      float ss = 0.0f;
#pragma unroll
      for (int i = 0; i < kXStaged; ++i) {
        const int t = static_cast<int>(threadIdx.x) + 64 * nq * i;
        const f32x4 a = stage.a[i], b = stage.b[i];
        if (t < K / 8)
          ss += ((a.x * a.x + a.y * a.y) + (a.z * a.z + a.w * a.w)) +
                ((b.x * b.x + b.y * b.y) + (b.z * b.z + b.w * b.w));
        stage.a[i] = a * nstage.a[i];
        stage.b[i] = b * nstage.b[i];
      }
      ss = row_lanes_sum<64>(ss);  // DPP and lane swaps: no LDS round trips
      if (lane == 0) norm_part[wave] = ss;
    }
  }
  if (wave < nq) quantize_staged_into_lds<1>(1, K, nq, stage, xq);  // K <= kStreamMaxK: all staged
  __syncthreads();
  float out_scale = 1.0f;
  if constexpr (MODE == 3) {
    float total = 0.0f;  // the waves' partials in wave order
    for (int i = 0; i < nq; ++i) total += norm_part[i];
    out_scale = rsqrtf(total / static_cast<float>(K) + eps);
  }

  // outputs in the global address space (the register copies above lost it)
  global_f32* gy = (global_f32*)(yout);
  global_f32* gh = (global_f32*)(hout);

  if constexpr (TYPE != 0) {
    stream_consume<TYPE, J, kFfn ? 1 : MODE, false, MODE == 3>(ws, S, max_sb, r0, r1, gy, gh, xq, wlds, sums, out_scale);
  } else {
    if (type == QK_TYPE_Q4_K)
      stream_consume<QK_TYPE_Q4_K, J, kFfn ? 1 : MODE, true, MODE == 3>(ws, S, max_sb, r0, r1, gy, gh, xq, wlds, sums, out_scale);
    else
      stream_consume<QK_TYPE_Q6_K, J, kFfn ? 1 : MODE, true, MODE == 3>(ws, S, max_sb, r0, r1, gy, gh, xq, wlds, sums, out_scale);
  }
}

using StreamKernel = void (*)(StreamParams);

}  // namespace qk
