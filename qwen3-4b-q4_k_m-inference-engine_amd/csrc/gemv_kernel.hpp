// Streaming Q4_K / Q6_K mat-vec kernel templates (M <= 8 activation rows).
//
// Replaces quantize + project<Q4_K/Q6_K> (src/cuda/matmul.cu:8-22, 86-125),
// which run one 128-thread block per output element after a separate
// quantize launch. Here one launch of 512-thread workgroups (8 waves, one
// workgroup per CU) does both:
//   1. prologue: every kernel argument is read in one scalar-load round; the
//      workgroup quantises the fp32 activations into Q8 blocks in LDS (or
//      copies caller-provided Q8 blocks) while each wave's first weight
//      loads are already in flight;
//   2. each wave64 is an independent worker over a flat stream of
//      iterations: lane = (row rr = lane / LPR, c = lane % LPR) with
//      c -> (superblock offset c/4, piece c%4), so one iteration covers
//      64/LPR rows x LPR/4 whole superblocks. Iterations run U at a time,
//      double buffered (the next U are loading while the current U are
//      consumed) across row-unit boundaries; the lanes of a row reduce with
//      DPP/shuffles when its last iteration is consumed. No barriers after
//      the prologue, and no load is ever issued under a branch, so the
//      compiler's wait counts stay exact.
// Several weight segments sharing the input (attn q/k/v, src/Engine.cpp:83-85)
// run in one launch; the FFN mode computes gate and up for the same rows and
// writes SiLU(gate)*up (src/Engine.cpp:98-100, src/cuda/silu_multiply.cu:10).
#pragma once

#include <type_traits>

#include "argmax.hpp"
#include "qk_device.hpp"
#include "qk_launch.hpp"

namespace qk {

// Waves per workgroup, iterations per chunk (Q4_K, Q6_K) and activation
// tasks staged per quantiser lane: the values measured best on the Qwen3-4B
// decode sweep. M > 1: 8 waves, several accumulators per lane in up to 256
// VGPRs. M = 1 on this kernel means a shape too large for the whole-share
// kernel (the lm_head: one long stream per wave), measured faster with 8
// waves each two Q6_K iterations deep (196 VGPRs; 16 waves that deep spill)
// than with 16 waves one iteration deep.
constexpr int kMatvecWavesMt = 8;
constexpr int kMatvecU4 = 2;
constexpr int kMatvecU6 = 1;
constexpr int kMatvecXStaged = 2;
constexpr int kMatvecWavesM1 = 8;
constexpr int kMatvecU6M1 = 2;
// Waves per workgroup for MT activation rows.
template <int MT>
constexpr int matvec_waves() {
  return MT == 1 ? kMatvecWavesM1 : kMatvecWavesMt;
}

// Per-lane register image of one iteration's piece.
template <int TYPE>
struct PieceOf {
  using type = Q6KPiece;
};
template <>
struct PieceOf<QK_TYPE_Q4_K> {
  using type = Q4KPiece;
};

template <int TYPE>
__device__ __forceinline__ typename PieceOf<TYPE>::type load_piece(const uint8_t* sb, uint32_t pc,
                                                                    int) {
  if constexpr (TYPE == QK_TYPE_Q4_K) return load_q4k_piece(sb, pc);
  else return load_q6k_piece(sb, pc);
}

template <int TYPE>
__device__ __forceinline__ float dot_piece(const typename PieceOf<TYPE>::type& w, const XFrag& xa,
                                           const XFrag& xb, uint32_t pc, int) {
  if constexpr (TYPE == QK_TYPE_Q4_K) return dot_q4k_piece(w, xa, xb, pc);
  else return dot_q6k_piece(w, xa, xb, pc);
}

// Q8 blocks a piece pairs with: Q4_K piece j -> sub-blocks 2j, 2j+1;
// Q6_K piece p (half h, parity r) -> groups 4h+r and 4h+r+2.
__device__ __forceinline__ int piece_block_a(uint32_t pc, int type) {
  return type == QK_TYPE_Q4_K ? static_cast<int>(2 * pc)
                              : static_cast<int>(4 * (pc >> 1) + (pc & 1u));
}
__device__ __forceinline__ int piece_block_step(int type) { return type == QK_TYPE_Q4_K ? 1 : 2; }

// Q8 of one group of 8 consecutive activations per lane; the 4 lanes of a
// quad form one 32-activation block. code = roundf(RN(x/amax)*127) and
// scale = RN(amax/127), as the reference computes them in float, with
// amax in [2^-64, 2^64] (every amax for which a code can be non-zero):
//  - 1/amax: v_rcp_f32 plus one FMA refinement, which equals the IEEE
//    reciprocal for every amax in that range (checked exhaustively on gfx950);
//  - x/amax and amax/127: Markstein's correction q0 = x*r, e = fma(-q0, b, x),
//    q = fma(e, r, q0) with the correctly rounded reciprocal r, which gives the
//    IEEE quotient (x/amax: checked on the CPU over 3.1e8 random and 9e6
//    near-tie pairs and on the GPU; amax/127: exhaustively on gfx950);
//  - roundf(t) for |t| <= 127: trunc(t + copysign(0.49999997f, t)), equal to
//    roundf for every such float (checked exhaustively); the float-to-int
//    conversion truncates.
// Other amax take the IEEE division and roundf. (refined_rcp, markstein_div
// and round_code live in qk_device.hpp; tests/cpp/quant_arith_check.hip
// repeats the exhaustive checks on the GPU.)

// One quad lane's share of a 32-value block: its 8 codes packed in two dwords,
// the block scale, and (from the quad's DPP sums) the sums of codes 0..15
// (pair) and 16..31 (other) as seen by lane 0 of the quad. Every lane of the
// quad must call it (the DPP exchanges read the neighbours).
struct Q8Quarter {
  uint32_t lo, hi;
  float scale;
  int pair, other;
};

__device__ __forceinline__ Q8Quarter quantize_quarter(const float (&v)[8]) {
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
  amax = fmaxf(amax, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                         0, __builtin_bit_cast(int, amax), 0xB1, 0xF, 0xF, false)));
  amax = fmaxf(amax, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                         0, __builtin_bit_cast(int, amax), 0x4E, 0xF, 0xF, false)));
  const bool usual = amax >= 0x1p-64f && amax <= 0x1p64f;
  int code[8];
  float scale;
  if (usual) {
    const float r = refined_rcp(amax);
#pragma unroll
    for (int i = 0; i < 8; ++i) code[i] = q8_code(v[i], amax, r);
    scale = markstein_div(amax, 127.0f, 1.0f / 127.0f);
  } else if (amax == 0.0f) {
#pragma unroll
    for (int i = 0; i < 8; ++i) code[i] = 0;
    scale = 0.0f;
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) code[i] = static_cast<int>(roundf((v[i] / amax) * 127.0f));
    scale = amax / 127.0f;
  }
  uint32_t lo = 0, hi = 0;
  int sum = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    lo |= (static_cast<uint32_t>(code[i]) & 0xFFu) << (8 * i);
    hi |= (static_cast<uint32_t>(code[i + 4]) & 0xFFu) << (8 * i);
    sum += code[i] + code[i + 4];
  }
  // lanes 0,1 of the quad hold codes 0..15, lanes 2,3 codes 16..31
  const int pair = sum + __builtin_amdgcn_update_dpp(0, sum, 0xB1, 0xF, 0xF, false);
  const int other = __builtin_amdgcn_update_dpp(0, pair, 0x4E, 0xF, 0xF, false);
  return Q8Quarter{lo, hi, scale, pair, other};
}

// Quarter `quarter` of a Q8 block record in global memory (qk_q8_block):
// its 8 codes, and from lane 0 of the quad the 16-byte tail (scale,
// scale * sum of codes, -32 * sums of codes 0..15 and 16..31).
__device__ __forceinline__ void store_q8_quarter(qk_q8_block* blk, uint32_t quarter, const Q8Quarter& q) {
  *reinterpret_cast<u32x2*>(blk->codes + 8 * quarter) = u32x2{q.lo, q.hi};
  if (quarter == 0) {
    const f32x4 rec = {q.scale, q.scale * static_cast<float>(q.pair + q.other),
                       __builtin_bit_cast(float, -32 * q.pair), __builtin_bit_cast(float, -32 * q.other)};
    *reinterpret_cast<f32x4*>(&blk->scale) = rec;
  }
}

__device__ __forceinline__ void quantize_group(const float (&v)[8], lds_q8_block* blk, uint32_t q) {
  const Q8Quarter r = quantize_quarter(v);
  *reinterpret_cast<lds_u32x2*>(blk->codes + 8 * q) = u32x2{r.lo, r.hi};
  if (q == 0) {
    blk->scale = r.scale;
    blk->scaled_sum = r.scale * static_cast<float>(r.pair + r.other);
    blk->neg32_sum_lo = -32 * r.pair;
    blk->neg32_sum_hi = -32 * r.other;
  }
}

// The prologue quantises fp32 x[M x K] into LDS Q8 blocks [MT][K/32] (rows
// m >= M are zero), 8 activations per task. Only the first nq waves of the
// workgroup (the quantiser waves) touch x: each of their lanes issues the
// loads of up to kXStaged tasks before its weight loads and quantises them
// while those are in flight. Global loads return in issue order per wave, so
// the other waves' weight loads never wait behind activation loads. Tasks
// beyond the staged ones (M > 1 with wide K) load and quantise afterwards.
constexpr int kXStaged = kMatvecXStaged;

template <int MT>
struct XStage {
  f32x4 a[kXStaged], b[kXStaged];
};

// Quantiser waves for `tasks` tasks: enough for kXStaged tasks per lane.
template <int MT>
__device__ __forceinline__ int quantiser_waves(int tasks) {
  return min(matvec_waves<MT>(), (tasks + 64 * kXStaged - 1) / (64 * kXStaged));
}

// Loads of every staged task are unconditional (indices clamped into the
// buffer, rows m >= M selected to zero afterwards).
__device__ __forceinline__ void load_x_group(const float* __restrict__ x, int M, int K, int t,
                                             f32x4& a, f32x4& b) {
  const int groups = K / 8;
  const int m = t / groups;
  const float* p = x + static_cast<int64_t>(min(m, M - 1)) * K + 8 * (t - m * groups);
  a = *reinterpret_cast<const f32x4_a4*>(p);
  b = *reinterpret_cast<const f32x4_a4*>(p + 4);
}

// Quantiser lane xl (threadIdx.x of a wave below nq) takes tasks xl + 64*nq*i.
template <int MT>
__device__ __forceinline__ void stage_x(const float* __restrict__ x, int M, int K, int nq,
                                        XStage<MT>& st) {
  const int tasks = MT * (K / 8);
#pragma unroll
  for (int i = 0; i < kXStaged; ++i) {
    const int t = min(static_cast<int>(threadIdx.x) + 64 * nq * i, tasks - 1);
    load_x_group(x, M, K, t, st.a[i], st.b[i]);
  }
}

__device__ __forceinline__ void quantize_task(f32x4 a, f32x4 b, bool zero, int t,
                                              lds_q8_block* lds) {
  if (zero) {
    a = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    b = a;
  }
  const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  // task t covers activations 8t..8t+7 of the [MT][K] stream: block t/4, quarter t%4
  quantize_group(v, lds + t / 4, static_cast<uint32_t>(t & 3));
}

// K/8 and 64*nq are multiples of 4, so the 4 lanes of a quad are always in
// or out together.
template <int MT>
__device__ __forceinline__ void quantize_staged_into_lds(int M, int K, int nq, const XStage<MT>& st,
                                                         lds_q8_block* lds) {
  const int groups = K / 8;
  const int tasks = MT * groups;
  const int step = 64 * nq;
#pragma unroll
  for (int i = 0; i < kXStaged; ++i) {
    const int t = static_cast<int>(threadIdx.x) + step * i;
    if (t < tasks) quantize_task(st.a[i], st.b[i], t / groups >= M, t, lds);
  }
}

template <int MT>
__device__ void quantize_into_lds(const float* __restrict__ x, int M, int K, int nq,
                                  const XStage<MT>& st, lds_q8_block* lds) {
  quantize_staged_into_lds<MT>(M, K, nq, st, lds);
  const int groups = K / 8;
  const int tasks = MT * groups;
  const int step = 64 * nq;
  for (int t = static_cast<int>(threadIdx.x) + step * kXStaged; t < tasks; t += step) {
    f32x4 a, b;
    load_x_group(x, M, K, t, a, b);
    quantize_task(a, b, t / groups >= M, t, lds);
  }
}

// Caller-provided Q8 blocks [M][K/32] -> LDS [MT][K/32]; rows m >= M are zero.
template <int MT>
__device__ void copy_q8_into_lds(const qk_q8_block* __restrict__ q8, int M, int K,
                                 lds_q8_block* lds) {
  const int per_row = (K / 32) * 3;  // 16-byte chunks
  const u32x4* src = reinterpret_cast<const u32x4*>(q8);
  lds_u32x4* dst = reinterpret_cast<lds_u32x4*>(lds);
  for (int t = threadIdx.x; t < MT * per_row; t += 64 * matvec_waves<MT>()) {
    const int m = t / per_row;
    dst[t] = m < M ? src[t] : u32x4{0u, 0u, 0u, 0u};
  }
}

// v + the same register of the lane selected by a DPP control (row-local).
template <int CTRL>
__device__ __forceinline__ float add_dpp(float v) {
  return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                                                   0xF, 0xF, false));
}

// v summed over lane bit 4 / lane bit 5 with the gfx950 lane-swap
// instructions (VALU, no LDS round trip). The two results of a swap are
// copied out as scalars before the bit casts: bit casting the subscripted
// elements directly made the compiler use the first result twice.
__device__ __forceinline__ float swap16_sum(float v) {
  const auto t = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, v),
                                                  __builtin_bit_cast(unsigned, v), false, false);
  const unsigned a = t[0], b = t[1];
  return __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b);
}
__device__ __forceinline__ float swap32_sum(float v) {
  const auto t = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, v),
                                                  __builtin_bit_cast(unsigned, v), false, false);
  const unsigned a = t[0], b = t[1];
  return __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b);
}

// Sum over the LPR lanes of each row (aligned lane groups); every lane of the
// group receives the sum.
template <int LPR>
__device__ __forceinline__ float row_lanes_sum(float v) {
  v = add_dpp<0xB1>(v);                             // lane bit 0 (quad_perm 1,0,3,2)
  v = add_dpp<0x4E>(v);                             // lane bit 1 (quad_perm 2,3,0,1)
  if constexpr (LPR >= 8) v = add_dpp<0x141>(v);    // lane bit 2 (row_half_mirror)
  if constexpr (LPR >= 16) v = add_dpp<0x140>(v);   // lane bit 3 (row_mirror)
  if constexpr (LPR >= 32) v = swap16_sum(v);       // lane bit 4
  if constexpr (LPR >= 64) v = swap32_sum(v);       // lane bit 5
  return v;
}

// Position of a wave's iteration in its stream: row group u (kRPU rows) and
// iteration k within it (FFN mode: k < ipu gate, else up).
struct Cursor {
  int u, k;
};

// Kernel arguments held in scalar registers.
struct MatvecArgs {
  const float* x;
  const qk_q8_block* q8;
  float* h;
  int M, K, S, nseg;
  MatvecSegment sg[kMaxSegments];
};


// One weight type's share of a launch: rows [row_lo, row_hi) of the
// concatenated segments, streamed by workgroups wg of nwg, in groups of kRPU
// rows with each row's LPR lanes covering LPR/4 superblocks per iteration.
// Returns the thread's best argmax key (argmax mode; 0 otherwise).
template <int MT, int LPR, int U, int MODE, int TYPE, bool Q8IN>
__device__ __forceinline__ uint64_t matvec_body(const MatvecArgs& a, int row_lo, int row_hi, int wg,
                                                int nwg, lds_q8_block* xq) {
  using Piece = typename PieceOf<TYPE>::type;
  constexpr int kRPU = 64 / LPR;  // rows per group
  constexpr int kSPI = LPR / 4;   // superblocks per iteration
  constexpr int kBytes = TYPE == QK_TYPE_Q4_K ? kQ4KBytes : kQ6KBytes;
  const int S = a.S, M = a.M, K = a.K, nseg = a.nseg;

  const uint32_t lane = threadIdx.x & 63u;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int rr = static_cast<int>(lane) / LPR;
  const uint32_t c = lane % LPR;
  const uint32_t pc = c & 3u;                // piece
  const int sbo = static_cast<int>(c >> 2);  // superblock offset within the iteration
  // Row groups of kRPU rows are dealt round-robin: group g goes to worker
  // g % nworkers, worker = wave*nwg + wg, so consecutive groups run on
  // different CUs and, at any moment, the whole GPU streams one compact
  // window of the matrix (DRAM rows stay open for many requests).
  const int nworkers = nwg * matvec_waves<MT>();
  const int wid = wave * nwg + wg;
  const int groups_total = (row_hi - row_lo + kRPU - 1) / kRPU;
  const int ngroups = wid < groups_total ? (groups_total - 1 - wid) / nworkers + 1 : 0;
  const int ipu = (S + kSPI - 1) / kSPI;  // iterations per weight row
  const int ipu_total = MODE == 1 ? 2 * ipu : ipu;
  const int T = ngroups * ipu_total;
  const int last_row = row_hi - 1;  // a valid row for idle loads
  auto group_row = [&](int u) {     // first row of this worker's u-th group
    return row_lo + (wid + u * nworkers) * kRPU;
  };

  // segment of a row, field by field (a struct picked by a runtime index
  // would be copied to scratch memory)
  struct Where {
    const uint8_t* w;
    float* y;
    int rows, local;
  };
  auto locate = [&](int row, int phase) {
    const int j = (nseg > 1 && row >= a.sg[1].row_begin) + (nseg > 2 && row >= a.sg[2].row_begin) +
                  (nseg > 3 && row >= a.sg[3].row_begin);
    auto pick = [j](auto f0, auto f1, auto f2, auto f3) {
      return j == 0 ? f0 : j == 1 ? f1 : j == 2 ? f2 : f3;
    };
    Where o;
    o.w = MODE == 1 && phase ? a.sg[1].w : pick(a.sg[0].w, a.sg[1].w, a.sg[2].w, a.sg[3].w);
    o.y = pick(a.sg[0].y, a.sg[1].y, a.sg[2].y, a.sg[3].y);
    o.rows = pick(a.sg[0].rows, a.sg[1].rows, a.sg[2].rows, a.sg[3].rows);
    o.local = row - pick(a.sg[0].row_begin, a.sg[1].row_begin, a.sg[2].row_begin, a.sg[3].row_begin);
    return o;
  };
  auto advance = [&](Cursor& cur) {
    if (++cur.k == ipu_total) {
      cur.k = 0;
      ++cur.u;
    }
  };
  // Loads of U iterations from `cur` on; iterations past the wave's stream
  // re-read its last one (in bounds, never consumed).
  auto issue = [&](Cursor& cur, Piece (&f)[U]) {
#pragma unroll
    for (int i = 0; i < U; ++i) {
      const bool live = cur.u < ngroups;
      const int k = live ? cur.k : ipu_total - 1;
      const int phase = MODE == 1 && k >= ipu;
      const int kk = phase ? k - ipu : k;
      const int row = min(group_row(live ? cur.u : max(ngroups - 1, 0)) + rr, last_row);
      const Where o = locate(row, phase);
      const int s = min(kk * kSPI + sbo, S - 1);
      f[i] = load_piece<TYPE>(o.w + (static_cast<int64_t>(o.local) * S + s) * kBytes, pc, TYPE);
      advance(cur);
    }
  };

  // The first U iterations' weights are requested before the activations are
  // quantised; a quantiser wave's activation loads go out just ahead of them.
  const int nq = quantiser_waves<MT>(MT * (K / 8));
  const bool quantiser = wave < nq;  // wave-uniform
  XStage<MT> stage;
  Piece fa[U], fb[U];
  Cursor ci{0, 0};
  if constexpr (!Q8IN)
    if (quantiser) stage_x<MT>(a.x, M, K, nq, stage);
  __builtin_amdgcn_sched_barrier(0);
  issue(ci, fa);
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (Q8IN) {
    copy_q8_into_lds<MT>(a.q8, M, K, xq);
  } else {
    if (quantiser) quantize_into_lds<MT>(a.x, M, K, nq, stage, xq);
  }
  __syncthreads();

  float acc[MT], up[MT];
#pragma unroll
  for (int m = 0; m < MT; ++m) acc[m] = up[m] = 0.0f;
  uint64_t best_key = 0;  // argmax mode
  Cursor cc{0, 0};
  const int blk_a = piece_block_a(pc, TYPE), blk_step = piece_block_step(TYPE);
  auto consume = [&](const Piece (&f)[U], int t0) {
#pragma unroll
    for (int i = 0; i < U; ++i) {
      if (t0 + i < T) {  // wave-uniform; no global loads inside
        const int phase = MODE == 1 && cc.k >= ipu;
        const int kk = phase ? cc.k - ipu : cc.k;
        const int s_raw = kk * kSPI + sbo;
        // LDS block index (< 2^16: the blocks fit in LDS). The mask lets the
        // compiler form the address with a 24-bit multiply-add; a 32-bit one
        // became v_mad_u64_u32 with an unrelated register as its high half,
        // and a wait for that register's pending weight load.
        const int blk = (min(s_raw, S - 1) * 8 + blk_a) & 0xFFFF;
        // A Q6_K piece is unpacked once for all MT rows, and the rows' LDS
        // reads go out two rows at a time (hoisted all at once, with the
        // codes recomputed per row, 10-14 VGPRs spilled at MT = 8).
        [[maybe_unused]] Q6KCodes cd;
        if constexpr (TYPE != QK_TYPE_Q4_K) cd = unpack_q6k_piece(f[i], pc);
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          const lds_q8_block* xr = xq + m * S * 8 + blk;
          float v;
          if constexpr (TYPE == QK_TYPE_Q4_K) v = dot_q4k_piece(f[i], load_x(xr), load_x(xr + blk_step), pc);
          else v = dot_q6k_codes(cd, load_x(xr), load_x(xr + blk_step));
          const float add = s_raw < S ? v : 0.0f;
          if (phase) up[m] += add;
          else acc[m] += add;
          if (MT > 1 && (m & 1)) __builtin_amdgcn_sched_barrier(0);
        }
        if (cc.k == ipu_total - 1) {  // the group's last iteration: reduce and store
          const int row = group_row(cc.u) + rr;
          const Where o = locate(min(row, last_row), 0);
          const bool store = c == 0 && row < row_hi;
          if constexpr (MODE == 0) {
#pragma unroll
            for (int m = 0; m < MT; ++m) acc[m] = row_lanes_sum<LPR>(acc[m]);
            if (store) {
#pragma unroll
              for (int m = 0; m < MT; ++m)
                if (m < M) o.y[static_cast<int64_t>(m) * o.rows + o.local] = acc[m];
            }
          } else if constexpr (MODE == 2) {
            acc[0] = row_lanes_sum<LPR>(acc[0]);
            if (store) {
              if (o.y) o.y[o.local] = acc[0];
              best_key = max_key(best_key, argmax_key(acc[0], static_cast<uint32_t>(o.local)));
            }
          } else {
#pragma unroll
            for (int m = 0; m < MT; ++m) {
              acc[m] = row_lanes_sum<LPR>(acc[m]);
              up[m] = row_lanes_sum<LPR>(up[m]);
            }
            if (store) {
#pragma unroll
              for (int m = 0; m < MT; ++m) {
                const float g = acc[m];
                if (m < M)
                  a.h[static_cast<int64_t>(m) * o.rows + o.local] = (g / (1.0f + expf(-g))) * up[m];
              }
            }
          }
#pragma unroll
          for (int m = 0; m < MT; ++m) acc[m] = up[m] = 0.0f;
        }
        advance(cc);
      }
    }
  };

  // Two buffers so the register arrays stay static: the next U iterations
  // load while the current U are consumed. The last chunk issues nothing
  // further, and every consume follows its own issue sequence in the code, so
  // the wait before it counts exactly the loads issued after its buffer.
  const int nchunks = (T + U - 1) / U;
  for (int chunk = 0; chunk < nchunks;) {
    if (chunk + 1 == nchunks) {
      consume(fa, chunk * U);
      break;
    }
    issue(ci, fb);
    consume(fa, chunk * U);
    ++chunk;
    if (chunk + 1 == nchunks) {
      consume(fb, chunk * U);
      break;
    }
    issue(ci, fa);
    consume(fb, chunk * U);
    ++chunk;
  }
  return best_key;
}

// MODE 0: y_j = x . W_j^T for every segment. MODE 1: segments 0/1 are gate
// and up of the same shape; h = SiLU(x . gate^T) * (x . up^T). MODE 2 (M = 1,
// one segment, lm_head): y (optional) and the index of its largest entry,
// reduced across the launch (src/Engine.cpp:106-111, src/cuda/argmax.cu).
// TYPE: the weight type of every segment, or 0 for a launch whose segments
// are Q4_K first, then Q6_K: workgroups below split_wg stream the Q4_K rows
// [0, split_row), the others the Q6_K rows, each with a body specialised to
// its type. Q8IN: activations arrive as Q8 blocks (q8) instead of fp32 (x).
template <int MT, int LPR, int MODE, int TYPE, bool Q8IN>
__global__ __launch_bounds__((64 * matvec_waves<MT>())) void matvec_kernel(const MatvecParams p) {
  extern __shared__ __align__(16) unsigned char lds_raw[];
  lds_q8_block* xq = (lds_q8_block*)(lds_raw);
  constexpr int U4 = kMatvecU4;
  constexpr int U6 = MT == 1 ? kMatvecU6M1 : kMatvecU6;

  MatvecArgs a;
  a.x = p.x;
  a.q8 = p.q8;
  a.h = p.h;
  a.M = p.M;
  a.K = p.K;
  a.S = p.S;
  a.nseg = p.nseg;
#pragma unroll
  for (int j = 0; j < kMaxSegments; ++j) a.sg[j] = p.seg[j];
  const int rows_total = p.rows_total, split_wg = p.split_wg, split_row = p.split_row;
  const int grid = static_cast<int>(gridDim.x);
  // Every argument (padding included, so no loaded register is recycled for
  // a later load) is consumed here: the scalar loads are issued together and
  // waited for once, instead of one round trip per use site.
  void* const argmax_ws = p.argmax_ws;
  uint32_t* const argmax_result = p.argmax_result;
  asm volatile("" ::"s"(a.x), "s"(a.q8), "s"(a.h), "s"(a.M), "s"(a.K), "s"(a.S), "s"(a.nseg),
               "s"(rows_total), "s"(split_wg), "s"(split_row), "s"(p.pad), "s"(grid),
               "s"(argmax_ws), "s"(argmax_result));
#pragma unroll
  for (int j = 0; j < kMaxSegments; ++j)
    asm volatile("" ::"s"(a.sg[j].w), "s"(a.sg[j].y), "s"(a.sg[j].rows), "s"(a.sg[j].type),
                 "s"(a.sg[j].row_begin), "s"(a.sg[j].pad));

  const int wg = static_cast<int>(blockIdx.x);
  if constexpr (TYPE != 0) {
    const uint64_t key = matvec_body<MT, LPR, TYPE == QK_TYPE_Q4_K ? U4 : U6, MODE, TYPE, Q8IN>(
        a, 0, rows_total, wg, grid, xq);
    if constexpr (MODE == 2) {
      __shared__ uint64_t keys[matvec_waves<MT>() + 1];
      argmax_finish(key, static_cast<ArgmaxWorkspace*>(argmax_ws), argmax_result, keys,
                    matvec_waves<MT>());
    }
  } else {
    if (wg < split_wg)
      matvec_body<MT, LPR, U4, MODE, QK_TYPE_Q4_K, Q8IN>(a, 0, split_row, wg, split_wg, xq);
    else
      matvec_body<MT, LPR, U6, MODE, QK_TYPE_Q6_K, Q8IN>(a, split_row, rows_total, wg - split_wg,
                                                         grid - split_wg, xq);
  }
}

using MatvecKernel = void (*)(MatvecParams);

// Kernel for MT activation rows, lanes per row `lpr`, mode, weight type
// (0 = Q4_K and Q6_K segments) and input kind; nullptr for a combination that
// is not built.
template <int MT>
MatvecKernel matvec_kernel_for(int lpr, int mode, int type, bool q8in) {
  auto pick = [&](auto lpr_c) -> MatvecKernel {
    constexpr int L = decltype(lpr_c)::value;
    if (q8in) {
      if (mode != 0) return nullptr;
      if (type == QK_TYPE_Q4_K) return &matvec_kernel<MT, L, 0, QK_TYPE_Q4_K, true>;
      if (type == QK_TYPE_Q6_K) return &matvec_kernel<MT, L, 0, QK_TYPE_Q6_K, true>;
      return nullptr;
    }
    if (mode == 1) {
      if (type == QK_TYPE_Q4_K) return &matvec_kernel<MT, L, 1, QK_TYPE_Q4_K, false>;
      if (type == QK_TYPE_Q6_K) return &matvec_kernel<MT, L, 1, QK_TYPE_Q6_K, false>;
      return nullptr;
    }
    if (mode == 2) {
      if constexpr (MT != 1) return nullptr;
      if (type == QK_TYPE_Q4_K) return &matvec_kernel<MT, L, 2, QK_TYPE_Q4_K, false>;
      if (type == QK_TYPE_Q6_K) return &matvec_kernel<MT, L, 2, QK_TYPE_Q6_K, false>;
      return nullptr;
    }
    if (type == QK_TYPE_Q4_K) return &matvec_kernel<MT, L, 0, QK_TYPE_Q4_K, false>;
    if (type == QK_TYPE_Q6_K) return &matvec_kernel<MT, L, 0, QK_TYPE_Q6_K, false>;
    return &matvec_kernel<MT, L, 0, 0, false>;
  };
  switch (lpr) {
    case 8: return pick(std::integral_constant<int, 8>{});
    case 16: return pick(std::integral_constant<int, 16>{});
    case 32: return pick(std::integral_constant<int, 32>{});
    case 64: return pick(std::integral_constant<int, 64>{});
    default: return nullptr;
  }
}

}  // namespace qk
