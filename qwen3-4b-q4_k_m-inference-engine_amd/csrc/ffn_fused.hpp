// The FFN block for one activation row in one launch:
//   h = SiLU(Q8(x') . gate^T) * (Q8(x') . up^T),  y = Q8(h) . down^T,
// x' = x or RMSNorm(x) (src/Engine.cpp:97-101: rms_norm(ffn_norm), matmul
// gate, matmul up, silu_multiply, matmul down; src/cuda/silu_multiply.cu:6-12).
//
// One workgroup per CU, two phases around a grid barrier:
//   A. the whole-share gate/up product of gemv_stream.hpp (MODE 1 or the
//      RMSNorm fold), each workgroup a contiguous range of h rows, stored with
//      agent-scope coherent stores;
//   B. every workgroup reads all of h back, quantises it into LDS and runs the
//      whole-share product of its range of down rows.
// The down weights do not depend on h: waves 0..14 issue their share of them
// (16-byte loads of a contiguous superblock run, as for gate/up) during phase
// A, once their gate/up chunks are in LDS, so they stream while phase A
// computes. (Issued after phase A's pieces instead, they were still being
// issued when wave 15 stored h, and its stores queued behind them: +1.4 us.)
// Wave 15 forms phase A's row totals, stores h and runs the grid barrier; its
// down "loads" re-read one chunk (every wave issues the same loads, so the
// compiler's wait counts stay exact), and since gfx950 counts stores and loads
// in one counter, the wait for its h stores to complete does not include the
// real down stream. For a Q6_K down, while the barrier is
// pending the other waves move their chunks to LDS and unpack their pieces
// into int8 codes in registers, so that after it only the integer dots with h
// remain (done after the barrier, the unpacking measured ~3 us of VALU per CU
// on the critical path).
//
// Grid barrier (no cache maintenance: every byte exchanged is written and read
// with agent-scope coherent accesses). Workgroup b belongs to group b % 8 (the
// XCD the dispatcher places it on); the first thread of each workgroup, once
// its h stores are complete, adds 1 to its group's counter; the last of a
// group adds 1 to the global counter; the last group resets the counters,
// advances the epoch and writes it into the 8 per-group release words, which
// each workgroup polls. Per-group counters keep the serialised atomics on one
// address to 32 (a single counter for 256 workgroups measured ~4 us from the
// last arrival to the release; this scheme ~1.7 us on MI355X). The wait is
// bounded: after spin_ticks of the 100 MHz real-time clock the workgroup sets
// the timeout word and goes on, writing NaN into its y rows (so a missed
// check shows in the outputs; the launch's other rows may be invalid too).
// Co-residency: the launcher sizes the grid to the CU count with LDS that
// admits one workgroup per CU.
#pragma once

#include "gemv_stream.hpp"

namespace qk {

// Barrier words in the caller's workspace, one 256-byte line each (uint32
// index = line * kSyncLine): epoch, timeout flag, global counter, 8 group
// counters, 8 release words.
constexpr int kSyncLine = 64;
constexpr int kSyncGroups = 8;
constexpr int kSyncEpoch = 0;
constexpr int kSyncTimeout = 1 * kSyncLine;
constexpr int kSyncGlobal = 2 * kSyncLine;
constexpr int kSyncGroup0 = 3 * kSyncLine;
constexpr int kSyncRelease0 = (3 + kSyncGroups) * kSyncLine;
constexpr size_t kFfnSyncBytes = 8192;
static_assert((3 + 2 * kSyncGroups) * kSyncLine * 4 <= kFfnSyncBytes, "barrier lines fit");

constexpr int kFfnHWaves = 1;  // the last wave: phase A's row totals, the h stores, the barrier

// Byte offset of phase B's down region: right after the Q8 of h, unless that
// would overlap phase A's superblock sums (and norm partials), which the h
// wave may still be reading while the other waves move their down chunks to
// LDS; then right after those sums. (The Q8 of h itself is written after the
// barrier, when every wave is past phase A.)
__host__ __device__ constexpr int ffn_down_offset(int S, int JG, int max_sb, int Sd, int JD) {
  const int q8 = 48;  // sizeof(qk_q8_block)
  const int sums_a = S * 8 * q8 + kStreamWaves * JG * 1024;
  const int sums_a_end = sums_a + 2 * max_sb * 4 + 4 * kStreamWaves;
  const int after_h = Sd * 8 * q8;
  return after_h + kStreamWaves * JD * 1024 <= sums_a ? after_h : sums_a_end;
}

struct FfnParams {
  const float* x;         // [K]
  const float* norm;      // RMSNorm scale [K] (NORM kernels)
  float* h;               // [N] SiLU(gate) * up
  float* y;               // [K] down output
  const uint8_t* gate;    // [N rows x K]
  const uint8_t* up;      // [N rows x K]
  const uint8_t* down;    // [K rows x N]
  uint32_t* sync;         // barrier words (kFfnSyncBytes)
  int32_t K, S, N, Sd;    // widths and their superblocks (S = K/256, Sd = N/256)
  int32_t per, rem;       // h rows per workgroup: per, the first rem one more
  int32_t dper, drem;     // y rows per workgroup
  int32_t max_sb, max_sbd;  // superblocks of the largest share: gate/up per part, down
  float eps;              // RMSNorm epsilon (NORM kernels)
  uint32_t spin_ticks;    // bound of the barrier wait (s_memrealtime ticks)
};

typedef __attribute__((address_space(1))) uint32_t global_u32;

__device__ __forceinline__ uint32_t load_agent(const global_u32* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_agent(global_u32* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The epoch of the last barrier on this workspace, as workgroup b's group
// release word holds it (every release writes all 8 of them): 256 workgroups
// reading one word at launch serialise on it, 8 words spread them.
__device__ __forceinline__ uint32_t last_epoch_of(const uint32_t* sync) {
  const int g = static_cast<int>(blockIdx.x) & (kSyncGroups - 1);
  return load_agent((const global_u32*)(sync) + kSyncRelease0 + g * kSyncLine);
}

// Thread 0 of a workgroup, once its workgroup's h stores are complete.
// Returns false if the wait timed out.
__device__ __forceinline__ bool grid_barrier(global_u32* sync, uint32_t epoch, uint32_t spin_ticks) {
  const int G = static_cast<int>(gridDim.x);
  const int g = static_cast<int>(blockIdx.x) & (kSyncGroups - 1);
  const uint32_t size_g = static_cast<uint32_t>((G + kSyncGroups - 1 - g) / kSyncGroups);
  const uint32_t groups = static_cast<uint32_t>(min(G, kSyncGroups));
  global_u32* counter = sync + kSyncGroup0 + g * kSyncLine;
  if (__hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == size_g - 1) {
    store_agent(counter, 0u);  // every member arrived: ready for the next launch
    if (__hip_atomic_fetch_add(sync + kSyncGlobal, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
        groups - 1) {
      store_agent(sync + kSyncGlobal, 0u);
      store_agent(sync + kSyncEpoch, epoch);
      for (int k = 0; k < kSyncGroups; ++k) store_agent(sync + kSyncRelease0 + k * kSyncLine, epoch);
    }
  }
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  const global_u32* release = sync + kSyncRelease0 + g * kSyncLine;
  while (load_agent(release) != epoch) {
    if (__builtin_amdgcn_s_memrealtime() - t0 > spin_ticks) {
      store_agent(sync + kSyncTimeout, 1u);
      return false;
    }
    __builtin_amdgcn_s_sleep(2);
  }
  return true;
}

// Loads of the quantiser tasks of h (8 values each) with agent-scope coherent
// 16-byte loads through a buffer descriptor whose range is h: tasks past N
// read zeros.
__device__ __forceinline__ void stage_h(const float* h, int N, int nq, XStage<1>& st) {
  const __amdgpu_buffer_rsrc_t rsrc =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(h), 0, N * 4, 0x00020000);
  constexpr int kSc1 = 16;  // cache policy: agent scope (sc1)
#pragma unroll
  for (int i = 0; i < kXStaged; ++i) {
    const int t = static_cast<int>(threadIdx.x) + 64 * nq * i;
    st.a[i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, 32 * t, 0, kSc1));
    st.b[i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, 32 * t + 16, 0, kSc1));
  }
}

// A lane's Q6_K down pieces unpacked, q = lane + 64 i (i < PD) of its wave's
// share (superblock q/4 of the share, piece q%4); lanes past the share redo
// its last piece and store nothing.
template <int PD>
struct DownCodes {
  Q6KCodes codes[PD];
  int s0;  // superblock within its row of piece 0 (piece i: + 16 i, mod Sd)
};

// JG: 16-byte chunks per lane of the gate/up share; JD: of the down share.
// PD (Q6_K down): pieces per lane unpacked ahead of h; 0 for a Q4_K down,
// whose share goes through the whole-share consume after the barrier.
template <int TG, int JG, int TD, int JD, int PD, bool NORM>
__global__ __launch_bounds__(64 * kStreamWaves) void ffn_fused_kernel(const FfnParams p) {
  extern __shared__ __align__(16) unsigned char lds_raw[];
  constexpr int kWpp = kStreamWaves / 2;  // phase A: waves 0-7 gate, 8-15 up
  constexpr int kDownWaves = kStreamWaves - kFfnHWaves;  // waves 0..14 hold the down share
  constexpr int kHWave = kDownWaves;                     // wave 15 stores h, runs the barrier
  constexpr int BG = TG == QK_TYPE_Q4_K ? kQ4KBytes : kQ6KBytes;
  constexpr int BD = TD == QK_TYPE_Q4_K ? kQ4KBytes : kQ6KBytes;
  constexpr bool kEarly = PD > 0;  // Q6_K down unpacked ahead of h
  // Gate/up chunks issued at entry; the rest go out after the activation
  // barrier. With every chunk issued at entry the activations, requested
  // first, still arrived ~3.3 us after entry (p50; ~1.1 us with no weight
  // loads at all): they queue behind the whole chip's weight requests. With 3
  // of 7 chunks ahead (and 4 after) the activation barrier falls earlier, and
  // phase A, which is VALU-bound from there, ends earlier: block 14.9-15.0 ->
  // 14.4-14.5 us, decode step 0.927 -> 0.913-0.916 ms (same process, two
  // interleaved runs; 1 of 7 measured slower, 2 of 7 between). The same split
  // made the small whole-share launches slower (attn_qkv 5.1 -> 5.4 us).
  constexpr int kGuEarly = (3 * JG + 6) / 7;
  static_assert(!kEarly || TD == QK_TYPE_Q6_K, "early unpacking is for Q6_K");
  // Every argument in one scalar-load round (see matvec_kernel).
  asm volatile("" ::"s"(p.x), "s"(p.norm), "s"(p.h), "s"(p.y), "s"(p.gate), "s"(p.up), "s"(p.down),
               "s"(p.sync));
  asm volatile("" ::"s"(p.K), "s"(p.S), "s"(p.N), "s"(p.Sd), "s"(p.per), "s"(p.rem), "s"(p.dper),
               "s"(p.drem), "s"(p.max_sb), "s"(p.max_sbd), "s"(p.eps), "s"(p.spin_ticks));
  __builtin_amdgcn_sched_barrier(0);
  const int K = p.K, N = p.N;
  const int lane = static_cast<int>(threadIdx.x & 63u);
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));

  // The activation loads of the quantiser waves go out first.
  const int nq = min(kStreamWaves, (K / 8 + 64 * kXStaged - 1) / (64 * kXStaged));
  XStage<1> stage, nstage;
  if (wave < nq) {
    stage_x<1>(p.x, 1, K, nq, stage);
    if constexpr (NORM) stage_x<1>(p.norm, 1, K, nq, nstage);
  }
  __builtin_amdgcn_sched_barrier(0);
  // The launch's epoch (only the barrier thread uses it), behind the
  // activation loads so that no activation wait includes this coherent load,
  // which misses every cache; unconditional (a branch around it made the
  // compiler wait for it at the branch's end), and the increment waits for
  // the barrier.
  const uint32_t last_epoch = last_epoch_of(p.sync);

  const int wg = static_cast<int>(blockIdx.x);
  int r0 = wg * p.per + min(wg, p.rem);
  int r1 = r0 + p.per + (wg < p.rem ? 1 : 0);
  int d0 = wg * p.dper + min(wg, p.drem);
  int d1 = d0 + p.dper + (wg < p.drem ? 1 : 0);
  // Values used after the barriers are held in registers: left as kernel
  // arguments, the compiler re-reads them from memory there (a round trip).
  int S = p.S, Sd = p.Sd, max_sb = p.max_sb, max_sbd = p.max_sbd, Kd = K;
  float* hout = p.h;
  float* yout = p.y;
  uint32_t* sync = p.sync;
  uint32_t spin = p.spin_ticks;
  asm volatile("" : "+s"(S), "+s"(Sd), "+s"(max_sb), "+s"(max_sbd), "+s"(hout), "+s"(yout), "+s"(r0),
               "+s"(r1), "+s"(d0), "+s"(d1), "+s"(sync), "+s"(spin), "+s"(Kd));
  float eps = 0.0f;
  if constexpr (NORM) {
    eps = p.eps;
    asm volatile("" : "+s"(eps));
  }

  // Phase A share: superblocks of this wave's part (gate or up) of rows [r0, r1).
  WaveShare<JG> wsg;
  wsg.part = wave / kWpp;
  {
    const int wv = wave % kWpp;
    const int nsb = (r1 - r0) * S;
    wsg.sb_a = nsb * wv / kWpp;
    wsg.sb_b = nsb * (wv + 1) / kWpp;
    issue_share<JG, 0, kGuEarly>(wsg, wsg.part ? p.up : p.gate, N, r0, S, BG, lane);
  }
  // Phase B share: superblocks of down rows [d0, d1) (row-major) for waves
  // 0..14. The loads go out once all of the wave's gate/up chunks are in
  // LDS (issued at entry they delayed the activations and the gate/up
  // bytes behind them). Wave 15's share is empty: its loads re-read the
  // activations' first 16 bytes, a cached line, so that its wait for its h
  // stores (which also waits for every earlier load of the wave) is not held
  // up by a line of the down stream. (The weight pointers stay arithmetic on
  // the kernel arguments so that the loads are global loads, whose waits
  // count in order.)
  WaveShare<JD> wsd;
  wsd.part = 0;
  {
    const int nsb = (d1 - d0) * Sd;
    wsd.sb_a = wave < kDownWaves ? nsb * wave / kDownWaves : 0;
    wsd.sb_b = wave < kDownWaves ? nsb * (wave + 1) / kDownWaves : 0;
  }
  auto issue_down = [&]() {
    const bool own = wave < kDownWaves;
    issue_share<JD>(wsd, own ? p.down : reinterpret_cast<const uint8_t*>(p.x), Kd, own ? d0 : 0, Sd,
                    BD, lane);
  };
  __builtin_amdgcn_sched_barrier(0);

  // ---- phase A: gate/up, as the whole-share kernel's MODE 1 / 3
  lds_q8_block* xq = (lds_q8_block*)(lds_raw);
  lds_u8* wlds = (lds_u8*)(lds_raw) + S * 8 * static_cast<int>(sizeof(qk_q8_block));
  lds_f32* sums = reinterpret_cast<lds_f32*>(wlds + kStreamWaves * JG * 1024);
  lds_f32* norm_part = sums + 2 * max_sb;
  if constexpr (NORM) {
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
      ss = row_lanes_sum<64>(ss);
      if (lane == 0) norm_part[wave] = ss;
    }
  }
  if (wave < nq) quantize_staged_into_lds<1>(1, K, nq, stage, xq);  // K <= kStreamMaxK: all staged
  __syncthreads();
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (kGuEarly < JG)  // the rest of the gate/up share
    issue_share<JG, kGuEarly, JG>(wsg, wsg.part ? p.up : p.gate, N, r0, S, BG, lane);
  __builtin_amdgcn_sched_barrier(0);
  float out_scale = 1.0f;
  if constexpr (NORM) {
    float total = 0.0f;  // the waves' partials in wave order
    for (int i = 0; i < nq; ++i) total += norm_part[i];
    out_scale = rsqrtf(total / static_cast<float>(K) + eps);
  }
  // (its last step: wave 15 forms the row totals and stores h)
  stream_consume<TG, JG, 1, true, NORM, true, kHWave, kFfnHWaves, JG - 1>(
      wsg, S, max_sb, r0, r1, nullptr, (global_f32*)(hout), xq, wlds, sums, out_scale, issue_down);

  // LDS of phase B: Q8 of h, the down regions of the waves (JD KB each) at
  // ffn_down_offset (clear of phase A's sums, which wave 15 may still be
  // reading), then the superblock sums.
  static_assert(sizeof(qk_q8_block) == 48, "Q8 block layout");
  lds_q8_block* hq = (lds_q8_block*)(lds_raw);
  lds_u8* dlds = (lds_u8*)(lds_raw) + ffn_down_offset(S, JG, max_sb, Sd, JD);
  lds_f32* dsums = reinterpret_cast<lds_f32*>(dlds + kStreamWaves * JD * 1024);
  DownCodes<kEarly ? PD : 1> dc;
  const int npc = 4 * (wsd.sb_b - wsd.sb_a);
  // the barrier's outcome for the whole workgroup, in phase A's norm
  // partials (dead by now; phase B's regions are clear of them)
  lds_u32* passed = reinterpret_cast<lds_u32*>(norm_part);
  if (wave == kHWave) {
    // ---- grid barrier: h complete everywhere (this wave stored all of it).
    // The wait is one inline-asm statement with a memory clobber, so the
    // compiler keeps every h store before it and the counter add after it.
    asm volatile("s_waitcnt vmcnt(0) expcnt(0) lgkmcnt(0)" ::: "memory");
    if (lane == 0) *passed = grid_barrier((global_u32*)(sync), last_epoch + 1u, spin) ? 1u : 0u;
  } else if constexpr (kEarly) {
    // Meanwhile the down waves move their chunks to LDS and unpack their
    // pieces (nothing of that depends on h).
    lds_u8* reg = dlds + wave * (JD * 1024);
#pragma unroll
    for (int j = 0; j < JD; ++j) {
      const int off = wsd.off(j, lane);
      lds_u32* d = reinterpret_cast<lds_u32*>(reg + off);
      if ((off & 15) == 0) {
        *reinterpret_cast<lds_u32x4*>(d) = wsd.chunk[j];
      } else {
        d[0] = wsd.chunk[j].x;
        d[1] = wsd.chunk[j].y;
        d[2] = wsd.chunk[j].z;
        d[3] = wsd.chunk[j].w;
      }
    }
    asm volatile("" ::: "memory");  // the wave's reads below follow its writes
#pragma unroll
    for (int i = 0; i < PD; ++i) {
      const int q = npc > 0 ? min(lane + 64 * i, npc - 1) : 0;
      const uint32_t pc = static_cast<uint32_t>(q) & 3u;
      dc.codes[i] = unpack_q6k_piece(lds_q6k_piece(reg + wsd.o + (q >> 2) * kQ6KBytes, pc), pc);
    }
    dc.s0 = (wsd.sb_a + (lane >> 2)) % Sd;  // superblock within its row of the first piece
  }
  __syncthreads();
  // A timed-out wait read h that may be another call's: this workgroup's y
  // rows become NaN (every other word of the outputs is still written).
  const float y_scale = *passed ? 1.0f : __builtin_nanf("");

  // ---- phase B: Q8 of h into LDS, then the down rows. Every wave takes
  // quantiser tasks (lane l of the workgroup tasks l, l + 1024): with the
  // fewest waves that stage all N / 8 tasks (10 for N = 9728, 2 tasks a lane)
  // one SIMD ran 6 tasks a lane, with all 16 at most 5 (block 15.6-15.8 ->
  // 15.5 us); phase A keeps its few quantiser waves, whose loads go out
  // ahead of the weight loads (all 16 there measured slower).
  constexpr int nqh = kStreamWaves;
  {
    XStage<1> hs;
    stage_h(hout, N, nqh, hs);
    quantize_staged_into_lds<1>(1, N, nqh, hs, hq);  // N <= kStreamMaxK: all staged
  }
  __syncthreads();
  if constexpr (kEarly) {
    if (wave < kDownWaves) {
      const uint32_t pc = static_cast<uint32_t>(lane) & 3u;
      const int blk_a = piece_block_a(pc, QK_TYPE_Q6_K);
      const int step = 16 % Sd;
      int s = dc.s0;
#pragma unroll
      for (int i = 0; i < PD; ++i) {
        const int q = lane + 64 * i;
        const lds_q8_block* xr = hq + ((s * 8 + blk_a) & 0xFFFF);
        float v = dot_q6k_codes(dc.codes[i], load_x(xr), load_x(xr + 2));
        v = add_dpp<0xB1>(v);
        v = add_dpp<0x4E>(v);
        if (pc == 0 && q < npc) dsums[wsd.sb_a + (q >> 2)] = v;
        s += step;
        if (s >= Sd) s -= Sd;
      }
    }
    __syncthreads();
    // Row totals, a quad per row: lane k of the quad adds the row's
    // superblock sums k, k+4, ... in order, then the quad's DPP sum (the
    // whole-share kernel's order, so y matches a separate down launch).
    const int nrows = d1 - d0;
    const int k = lane & 3;
    for (int i = static_cast<int>(threadIdx.x) >> 2; i < nrows; i += 16 * kStreamWaves) {
      float g = 0.0f;
      for (int t = k; t < Sd; t += 4) g += dsums[i * Sd + t];
      g = add_dpp<0x4E>(add_dpp<0xB1>(g));
      if (k == 0) ((global_f32*)(yout))[d0 + i] = g * y_scale;
    }
  } else {
    stream_consume<TD, JD, 0, false, true>(wsd, Sd, max_sbd, d0, d1, (global_f32*)(yout), nullptr, hq, dlds,
                                           dsums, y_scale);
  }
}

using FfnKernel = void (*)(FfnParams);

}  // namespace qk
