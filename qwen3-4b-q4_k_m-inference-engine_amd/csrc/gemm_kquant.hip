// Q4_K / Q6_K dequantize-GEMM for prefill (M > 8 activation rows) on MFMA,
// with integer-structured weight operands.
//
// Replaces project<Q4_K/Q6_K> launched with gridDim.y = rows
// (src/cuda/matmul.cu:151-158). The activations arrive prepared (gemm.hip,
// prep_rows_kernel): v = 2^s(m) x8 with x8 the Q8 round trip of x
// (MatmulReference.hpp:11-29), held as fp16 planes hi + lo (22 significant
// bits), and for Q4_K X[m,j] = 2^-5 * (sum of v over 32-value block j), also
// as hi + lo. Every MFMA (v_mfma_f32_32x32x16_f16, fp32 accumulation) takes an
// activation plane as A and an exact fp16 integer weight operand as B:
//
// Q4_K (w = d*sc_j*q - dmin*m_j, src/cuda/embedding.cu:6-32): each superblock
// of a weight row adds d * sum_k v*(sc_j*q) - 32*dmin * sum_j m_j*X_j to
// 2^s*y. sc_j*q <= 63*15 is exact in fp16, so a 16-deep step is hi*B + lo*B;
// d and dmin fold in once per superblock and the min term is one more MFMA
// per superblock (A = X hi in k 0-7 and X lo in k 8-15, B = m_j in both).
//
// Q6_K (w = d*sc*q, q in -32..31, sc int8, src/cuda/embedding.cu:34-59):
// |sc*q| <= 4096, past the 2048 up to which fp16 integers are exact, so the
// operand is B_hi = fp16(sc*q) plus the exact remainder B_lo = sc*q - B_hi in
// {-1, 0, 1}: a step is hi*B_hi + lo*B_hi + hi*B_lo; d folds in once per
// superblock.
//
// Workgroup: 4 waves side by side in N, each owning TM x TN tiles of 32 x 32
// of the (BM = 32 TM) x (BN = 128 TN) output tile. K runs in stages of 64
// weights. Q4_K stage g of a superblock is its qs group g (sub-blocks 2g and
// 2g+1, low and high nibbles); Q6_K stage g is groups a and a+2 (a = g & 1)
// of half g / 2, which share their qh bytes.
//   - The activation tile of a stage (BM rows x hi/lo x the stage's 64
//     halves) goes through one of two LDS slots: the workgroup loads stage
//     c+2 into registers while it computes stage c and writes stage c+1
//     (loaded a stage earlier) in the middle of it; one barrier per stage.
//   - Each lane loads its own weight bytes into registers (a stage's 16 qs,
//     or 16 ql + 16 qh, bytes a stage ahead; a superblock's header or scales
//     and d during the superblock before) and, for Q4_K, its block sums once
//     per superblock: no weight tile passes through LDS.
//   - A grid of few tiles with a deep K splits K into superblock ranges;
//     gemm_kq_reduce_kernel adds the partial tiles in split order.
// Rows past M or N are clamped to the last row on load and not stored.
//
// MFMA operand rule (checked on the device): lane l gives row l%32 of A and
// column l%32 of B with the same 8 k values, half-wave l/32 choosing which 8;
// D lane l, register r holds row 8*(r/4) + 4*(l/32) + r%4, column l%32. The k
// order inside a step is free as long as A and B agree: in step (u, s) of a
// stage, half-wave h takes weights l = 16h + 8s .. +7 of its 32-weight group
// u (Q4_K: qs bytes 16h + 8s .. +7, nibble u; Q6_K: group a + 2u). An A slot
// row is 256 bytes, the 8 hi and 8 lo 16-byte pieces, piece L = 8*plane + p
// at position L ^ (row & 15), so the 16 rows a ds_read_b128 serves at once
// hit 16 different bank groups.
#include <algorithm>

#include "gemm_prep.hpp"
#include "qk_launch.hpp"

namespace qk {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) uint8_t lds_byte;
typedef __attribute__((address_space(3))) half8 lds_half8;
typedef __attribute__((address_space(3))) u32x4 lds_u32x4_t;

constexpr int kWaves = 4;
constexpr int kStageK = 64;  // weights of K per stage

template <int TM, int TN>
struct KQCfg {
  static constexpr int BM = 32 * TM;
  static constexpr int BN = 32 * TN * kWaves;
  static constexpr int SLOT = BM * 2 * 2 * kStageK;         // BM rows of hi + lo, 64 halves each
  static constexpr int PIECES = SLOT / 16 / (64 * kWaves);  // 16-byte A pieces per thread
  static_assert(PIECES >= 1 && SLOT % (16 * 64 * kWaves) == 0, "whole pieces per thread");
};

constexpr int kKQMaxSegments = 4;

struct KQGemmArgs {
  const float* x;      // short prompts (M <= kShortM): the activations [M x K] themselves
  const _Float16* hi;  // [M x K]; lo follows at + M*K
  const _Float16* xs;  // sub-block sums: [M][S][hi 8, lo 8] (Q4_K only)
  const float* row_scale;
  int32_t M, K, S, nseg;
  float* part;  // splits > 1 (one matrix): unscaled partial products [splits][M][N]
  int32_t n_tiles, tiles, per_xcd, splits;
  // The weight matrices of the launch (several share one split-free launch:
  // attn q, k and v of one activation tile): matrix j covers n-tiles
  // [tile0[j], tile0[j+1]) and writes y[j] [M x N[j]].
  const uint8_t* w[kKQMaxSegments];
  float* y[kKQMaxSegments];
  int32_t N[kKQMaxSegments], type[kKQMaxSegments], tile0[kKQMaxSegments];
};

// 8 weights (bytes of dwords lo, hi; nibble U) -> fp16 sc*q.
// (1024 + q) is the fp16 with bits 0x6400 | q; one fused multiply-add
// (1024 + q)*sc - 1024*sc gives sc*q exactly (U = 1 holds 16q in the byte:
// (1024 + 16q)*(sc/16) - 64*sc).
template <int U>
__device__ __forceinline__ half8 weights_fp16(uint32_t lo, uint32_t hi, half2v c, half2v e) {
  constexpr uint32_t mask = U ? 0xF0F0F0F0u : 0x0F0F0F0Fu;
  const uint32_t a = lo & mask, b = hi & mask;
  auto pair = [&](uint32_t v, uint32_t sel) {
    const half2v h = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, v, sel));
    return __builtin_elementwise_fma(h, c, e);
  };
  const half2v p0 = pair(a, 0x04010400u), p1 = pair(a, 0x04030402u);
  const half2v p2 = pair(b, 0x04010400u), p3 = pair(b, 0x04030402u);
  return half8{p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
}

// 8 Q6_K weights (ql bytes of dwords l0/l1, nibble U; qh bytes of h0/h1,
// bits shift..shift+1) -> fp16 sc*q as hi + exact lo. Each byte's 6-bit code
// c becomes the fp16 1024 + c (bits 0x6400 | c); minus 1056 gives q exactly;
// q*sc rounds once to hi and fma(q, sc, -hi) is the exact remainder.
template <int U>
__device__ __forceinline__ void weights_q6k(uint32_t l0, uint32_t l1, uint32_t h0, uint32_t h1,
                                            uint32_t shift, half2v sc, half8& bh, half8& bl) {
  auto code = [shift](uint32_t l, uint32_t hb) {
    return ((U ? l >> 4 : l) & 0x0F0F0F0Fu) | (((hb >> shift) & 0x03030303u) << 4);
  };
  const uint32_t c0 = code(l0, h0), c1 = code(l1, h1);
  half2v q[4];
  const uint32_t sel[2] = {0x04010400u, 0x04030402u};
#pragma unroll
  for (int i = 0; i < 4; ++i)
    q[i] = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, i < 2 ? c0 : c1, sel[i & 1])) +
           half2v{-1056.0f16, -1056.0f16};
  half2v hi[4], lo[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    hi[i] = q[i] * sc;
    lo[i] = __builtin_elementwise_fma(q[i], sc, -hi[i]);
  }
  bh = half8{hi[0].x, hi[0].y, hi[1].x, hi[1].y, hi[2].x, hi[2].y, hi[3].x, hi[3].y};
  bl = half8{lo[0].x, lo[0].y, lo[1].x, lo[1].y, lo[2].x, lo[2].y, lo[3].x, lo[3].y};
}

// One output tile (m-tile mt, n-tile nt of matrix wmat [N rows]) of one K
// split; `slots` is the workgroup's activation staging.
template <int TYPE, int TM, int TN>
__device__ __forceinline__ void kq_tile(const KQGemmArgs& args, uint8_t (&slots)[2][KQCfg<TM, TN>::SLOT],
                                        int mt, int nt, int split, const uint8_t* wmat, float* ymat,
                                        int N) {
  using C = KQCfg<TM, TN>;
  constexpr bool kQ6 = TYPE == QK_TYPE_Q6_K;
  constexpr int B = kQ6 ? kQ6KBytes : kQ4KBytes;  // superblock bytes
  constexpr int QW = kQ6 ? 2 : 1;                 // 16-byte weight loads per stage and n-tile
  const int m0 = mt * C::BM, n0 = nt * C::BN;
  const int M = args.M, K = args.K, S = args.S;
  const int sb0 = split * S / args.splits, sb1 = (split + 1) * S / args.splits;
  const int c_last = 4 * sb1 - 1;  // loads past the split's end re-read its last stage

  const int tid = static_cast<int>(threadIdx.x);
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = lane >> 5, l32 = lane & 31;

  // Activation pieces of this thread: f = tid + 256 v -> row f / 16,
  // position f % 16 holding piece L = (f % 16) ^ (row & 15) of plane L / 8;
  // piece p = L % 8 of a stage is its 8 halves at stage-local k 8p (Q4_K:
  // the stage is k 64c .. 64c+63) or 64 (p / 4) + 8 (p % 4) (Q6_K: groups
  // a and a+2 of a superblock half); LDS byte 16 f.
  const _Float16* pa[C::PIECES];
#pragma unroll
  for (int v = 0; v < C::PIECES; ++v) {
    const int f = tid + 64 * kWaves * v;
    const int row = f >> 4, piece = (f & 15) ^ (row & 15), p = piece & 7;
    pa[v] = args.hi + (piece >> 3 ? static_cast<int64_t>(M) * K : 0) +
            static_cast<int64_t>(min(m0 + row, M - 1)) * K + (kQ6 ? 64 * (p >> 2) + 8 * (p & 3) : 8 * p);
  }
  // first halves of stage c: Q4_K 64c; Q6_K 256 sb + 128 (half) + 32 a
  auto stage_k = [](int c) {
    return kQ6 ? 256 * (c >> 2) + 128 * ((c >> 1) & 1) + 32 * (c & 1) : kStageK * c;
  };
  // Weight rows of this lane (one per n-tile) and sub-block sum rows (one per m-tile).
  const uint8_t* wrow[TN];
#pragma unroll
  for (int j = 0; j < TN; ++j)
    wrow[j] = wmat +
              static_cast<int64_t>(min(n0 + wave * 32 * TN + 32 * j + l32, N - 1)) * S * B;
  // The sub-block sum row of m-tile i is formed where it is used: a pointer
  // held across the superblock loop is a register the 64-row tile cannot
  // spare (the compiler hoisted it out of the loop and spilled it there; the
  // lane index read through asm keeps the computation at its use).
  auto xrow = [&](int i) {
    int t;
    asm volatile("v_and_b32 %0, 63, %1" : "=v"(t) : "v"(static_cast<int>(threadIdx.x)));
    return args.xs + static_cast<int64_t>(min(m0 + 32 * i + (t & 31), M - 1)) * S * 16 + 8 * (t >> 5);
  };

  auto load_a = [&](int c, u32x4 (&r)[C::PIECES]) {
#pragma unroll
    for (int v = 0; v < C::PIECES; ++v) r[v] = load16(pa[v] + stage_k(c));
  };
  auto store_a = [&](int slot, const u32x4 (&r)[C::PIECES]) {
#pragma unroll
    for (int v = 0; v < C::PIECES; ++v)
      *reinterpret_cast<lds_u32x4_t*>((lds_byte*)slots[slot] + 16 * (tid + 64 * kWaves * v)) = r[v];
  };
  // This lane's weight bytes. Per superblock: Q4_K its header (d, dmin, 12
  // scale bytes); Q6_K its 16 scales and d (superblocks are 2-byte aligned).
  // Per stage c = 4 sb + g: Q4_K qs bytes 32g + 16h .. +15; Q6_K ql bytes
  // 64 (g/2) + 32 (g%2) + 16h .. +15 and qh bytes 32 (g/2) + 16h .. +15.
  auto load_head = [&](int sb, u32x4 (&hd)[TN], uint32_t (&dd)[TN]) {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const uint8_t* p = wrow[j] + sb * B;
      if constexpr (kQ6) {
        hd[j] = load16_a2(p + 192);
        dd[j] = load_u16(p + 208);
      } else {
        hd[j] = load16(p);
        dd[j] = 0;
      }
    }
  };
  auto load_q = [&](int c, u32x4 (&q)[TN][QW]) {
    const int g = c & 3;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const uint8_t* p = wrow[j] + (c >> 2) * B;
      if constexpr (kQ6) {
        q[j][0] = load16_a2(p + 64 * (g >> 1) + 32 * (g & 1) + 16 * h);
        q[j][1] = load16_a2(p + 128 + 32 * (g >> 1) + 16 * h);
      } else {
        q[j][0] = load16(p + 16 + 32 * g + 16 * h);
      }
    }
  };
  auto load_x = [&](int sb, u32x4 (&x)[TM]) {
#pragma unroll
    for (int i = 0; i < TM; ++i) x[i] = load16(xrow(i) + 16 * sb);
  };

  // acc: the output tile; ph: this superblock's products, both activation
  // planes (and for Q6_K the weight remainder) accumulated into one chain per
  // tile (a second accumulator per tile cost 32 VGPRs at TM = 2, the margin
  // between two and three workgroups per CU)
  f32x16 acc[TM][TN], ph[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = ph[i][j][r] = 0.0f;

  // In flight across stages: areg (activations, loaded in stage c-1 and
  // stored to LDS in stage c for stage c+1), bq[p] (qs bytes of the stages of
  // parity p, loaded a stage ahead), wh[p] (headers of the superblocks of
  // parity p, loaded during the superblock before) and xa (this superblock's
  // sub-block sums, loaded in its stage 2). Every loaded dword is used, so no load destination is
  // recycled early, and the superblock loop is unrolled by two so no loaded
  // register is copied at the loop edge.
  u32x4 areg[C::PIECES], wh[2][TN], bq[2][TN][QW], xa[TM];
  uint32_t wd[2][TN];
  load_a(4 * sb0, areg);
  load_head(sb0, wh[0], wd[0]);
  load_q(4 * sb0, bq[0]);
  store_a(0, areg);
  load_a(min(4 * sb0 + 1, c_last), areg);
  __syncthreads();

  const int swz = l32 & 15;  // row & 15 of every A row this lane reads
  auto superblock = [&](int sb, const u32x4 (&hcur)[TN], const uint32_t (&dcur)[TN],
                        u32x4 (&hnext)[TN], uint32_t (&dnext)[TN]) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int c = 4 * sb + g;
      load_q(min(c + 1, c_last), bq[(g + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);  // nothing of stage c+1 moves above stage c's work

      // weight-side constants. Q4_K: of sub-blocks 2g (nibble 0) and 2g+1
      // (nibble 1); Q6_K: the scales of groups a and a+2 for this lane's l
      // (index 8 (g/2) + 2 (a + 2U) + h: byte 2a + h of dword 2 (g/2) + U)
      half2v cm[TN][2], ce[TN][2];
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const u32x4 hd = hcur[j];
        if constexpr (kQ6) {
#pragma unroll
          for (int U = 0; U < 2; ++U) {
            const int sc = __builtin_amdgcn_sbfe(static_cast<int>(hd[2 * (g >> 1) + U]),
                                                 8 * (2 * (g & 1)) + 8 * h, 8);
            const _Float16 sh = static_cast<_Float16>(static_cast<int16_t>(sc));
            cm[j][U] = half2v{sh, sh};
          }
          continue;
        }
        int sc0, mn0, sc1, mn1;
        scale_min_k4(2 * g, hd.y, hd.z, hd.w, sc0, mn0);
        scale_min_k4(2 * g + 1, hd.y, hd.z, hd.w, sc1, mn1);
        const _Float16 s0 = static_cast<_Float16>(static_cast<uint16_t>(sc0));
        const _Float16 s1 = static_cast<_Float16>(static_cast<uint16_t>(sc1));
        cm[j][0] = half2v{s0, s0};
        ce[j][0] = cm[j][0] * half2v{-1024.0f16, -1024.0f16};
        const half2v t1{s1, s1};
        cm[j][1] = t1 * half2v{0.0625f16, 0.0625f16};
        ce[j][1] = t1 * half2v{-64.0f16, -64.0f16};
        (void)mn0;  // the mins enter at the superblock's end
        (void)mn1;
      }

      // Steps: the MFMAs of step s interleaved with the weight conversion of
      // step s+1 and the A fragment reads of step s+kAB (kAB fragment
      // buffers: two for one m-tile; one at TM = 2, where the second buffer's
      // 16 VGPRs would hold the kernel to two workgroups per CU); the stage's
      // activation staging (store of stage c+1, loads of stage c+3) sits
      // between steps 1 and 2, under their MFMAs.
      const lds_byte* a_row = (const lds_byte*)slots[g & 1] + l32 * 256;
      auto read_a = [&](int step, half8 (&ah)[TM], half8 (&al)[TM]) {
        const int p = 4 * (step >> 1) + 2 * h + (step & 1);
#pragma unroll
        for (int i = 0; i < TM; ++i) {
          ah[i] = *reinterpret_cast<const lds_half8*>(a_row + 32 * i * 256 + 16 * (p ^ swz));
          al[i] = *reinterpret_cast<const lds_half8*>(a_row + 32 * i * 256 + 16 * ((8 + p) ^ swz));
        }
      };
      // bw: the weight operand (Q6_K: bw = hi, bx = exact remainder)
      auto convert = [&](int step, half8 (&bw)[TN], half8 (&bx)[TN]) {
        const int U = step >> 1, s = step & 1;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const u32x4 q = bq[g & 1][j][0];
          if constexpr (kQ6) {
            const u32x4 qh = bq[g & 1][j][QW - 1];
            if (U)
              weights_q6k<1>(q[2 * s], q[2 * s + 1], qh[2 * s], qh[2 * s + 1], 2 * (g & 1) + 4, cm[j][1], bw[j], bx[j]);
            else
              weights_q6k<0>(q[2 * s], q[2 * s + 1], qh[2 * s], qh[2 * s + 1], 2 * (g & 1), cm[j][0], bw[j], bx[j]);
          } else {
            bw[j] = U ? weights_fp16<1>(q[2 * s], q[2 * s + 1], cm[j][1], ce[j][1])
                      : weights_fp16<0>(q[2 * s], q[2 * s + 1], cm[j][0], ce[j][0]);
          }
        }
      };
      constexpr int kAB = TM >= 2 ? 1 : 2;
      half8 ah[kAB][TM], al[kAB][TM], bw[2][TN], bx[2][TN];
      read_a(0, ah[0], al[0]);
      if constexpr (kAB == 2) read_a(1, ah[1], al[1]);
      convert(0, bw[0], bx[0]);
#pragma unroll
      for (int step = 0; step < 4; ++step) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j) {
            const int ab = step % kAB;
            ph[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[ab][i], bw[step & 1][j], ph[i][j], 0, 0, 0);
            ph[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[ab][i], bw[step & 1][j], ph[i][j], 0, 0, 0);
            if constexpr (kQ6)
              ph[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[ab][i], bx[step & 1][j], ph[i][j], 0, 0, 0);
          }
        if (step < 3) convert(step + 1, bw[(step + 1) & 1], bx[(step + 1) & 1]);
        if (step + kAB < 4) read_a(step + kAB, ah[step % kAB], al[step % kAB]);
        if (step == 1) {
          // stage c+1's activations (loaded a stage ago) into the other
          // slot, then start loading stage c+2 into the same registers
          store_a((g + 1) & 1, areg);
          load_a(min(c + 2, c_last), areg);
          // the next superblock's headers, issued after this stage's
          // activation loads (vector loads complete in order: the next
          // stage's wait for activations does not wait for these)
          if (g == 2) load_head(min(sb + 1, sb1 - 1), hnext, dnext);
          if (!kQ6 && g == 2) load_x(sb, xa);
        }
        // one MFMA, then a share of the VALU and LDS work, repeated
#pragma unroll
        for (int k = 0; k < (kQ6 ? 3 : 2) * TM * TN; ++k) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x002, kQ6 ? 5 : 3, 0);
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
      }

      if (kQ6 && g == 3) {  // superblock end: acc += d * part
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j) {
            const float d = half_bits_to_float(dcur[j]);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              acc[i][j][r] = fmaf(d, ph[i][j][r], acc[i][j][r]);
              ph[i][j][r] = 0.0f;
            }
          }
      }
      if (!kQ6 && g == 3) {  // superblock end: acc += d * part - 32 dmin * (X . m)
        float dd[TN], dm[TN];
        u32x4 min_b[TN];  // m_j of the 8 sub-blocks as fp16 (formed here: short-lived)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          dd[j] = half_bits_to_float(hcur[j].x & 0xFFFFu);
          dm[j] = -32.0f * half_bits_to_float(hcur[j].x >> 16);
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            int sa, ma, sb2, mb;
            scale_min_k4(2 * q, hcur[j].y, hcur[j].z, hcur[j].w, sa, ma);
            scale_min_k4(2 * q + 1, hcur[j].y, hcur[j].z, hcur[j].w, sb2, mb);
            const half2v mm{static_cast<_Float16>(static_cast<uint16_t>(ma)),
                            static_cast<_Float16>(static_cast<uint16_t>(mb))};
            min_b[j][q] = __builtin_bit_cast(uint32_t, mm);
          }
        }
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j) {
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = fmaf(dd[j], ph[i][j][r], acc[i][j][r]);
            f32x16 zero;
#pragma unroll
            for (int r = 0; r < 16; ++r) zero[r] = 0.0f;
            ph[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                __builtin_bit_cast(half8, xa[i]), __builtin_bit_cast(half8, min_b[j]), zero, 0, 0, 0);
          }
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              acc[i][j][r] = fmaf(dm[j], ph[i][j][r], acc[i][j][r]);
              ph[i][j][r] = 0.0f;
            }
      }
      __builtin_amdgcn_sched_barrier(0);
      __syncthreads();
    }
  };
  for (int sb = sb0; sb < sb1; sb += 2) {
    superblock(sb, wh[0], wd[0], wh[1], wd[1]);
    if (sb + 1 < sb1) superblock(sb + 1, wh[1], wd[1], wh[0], wd[0]);
  }

  // epilogue: y = acc * 2^-s(m), or the unscaled partial of this split. The
  // lane's half and column come from the lane id again here (mbcnt), so no
  // register is held across the superblock loop for them (the 64-row Q4_K
  // tile spilled three there).
  const int el = static_cast<int>(__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)));
  const int eh = el >> 5, el32 = el & 31;
  float* const part = args.part + static_cast<int64_t>(split) * M * N;
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int m = m0 + 32 * i + 8 * (r >> 2) + 4 * eh + (r & 3);
      if (m >= M) continue;
      const float rs = args.row_scale[m];
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int n = n0 + wave * 32 * TN + 32 * j + el32;
        if (n >= N) continue;
        if (args.splits == 1)
          ymat[static_cast<int64_t>(m) * N + n] = acc[i][j][r] * rs;
        else
          part[static_cast<int64_t>(m) * N + n] = acc[i][j][r];
      }
    }
}

// ---- short prompts (M <= kShortM): one row of 32-row tiles, prep inside ----
//
// At M <= 32 a projection was three launches (prep, GEMM, split reduce), two of
// them fixed cost. Here each work unit forms the planes of its own K range
// itself, one superblock at a time, with a power-of-two scale per (row,
// superblock): the superblock's max |x| brought into [2^14, 2^15), the Q8
// round trip and hi/lo split of the prep kernel (gemm_prep.hpp) otherwise,
// and 2^-s folded into the superblock's d (and dmin) instead of a row scale
// at the end. Power-of-two scaling commutes with every rounding while no
// value is subnormal, so the outputs are the row-scaled ones bit for bit
// except where an fp16 plane value or the block sum of a row's far smaller
// superblock would underflow (there this form keeps more bits). All four
// stages of the superblock sit in LDS at once, so the stages run without
// barriers; the next superblock's activations are in flight meanwhile.
// Every n-tile forms the planes of its K range again, so the launch takes this
// form only for products of at most kGemmShortTiles n-tiles (gemm_short_plan).
// Measured at M = 23 (graph replays, against prep + GEMM (+ reduce)): attn_k
// 11.1 -> 9.3 us, attn_v 12.7 -> 10.8, attn_q 14.3 -> 13.1, attn_output
// 14.4 -> 13.2, ffn_down 31.2 -> 30.3; ffn_gate (76 n-tiles) 20.4 -> 21.7 and
// the lm_head (1187) 165 -> 195, so those keep the prep launch.
constexpr int kShortM = static_cast<int>(kGemmShortRows);

struct KQShortSmem {
  uint8_t a[4][32 * 256];  // the superblock's 4 stages: 32 rows of 8 hi + 8 lo 16-byte pieces (swizzled)
  _Float16 xs[32][16];     // Q4_K: per row, 2^-5 x the 8 sub-block sums of v, hi then lo
  float rs[32];            // per row: 2^-s of the superblock's scale
};

// Thread tid: row tid / 8, 32-value block tid % 8 of the superblock, whose
// values xv holds. Writes the block's hi and lo pieces where the staging of
// the prepared planes puts them (piece p of plane L / 8 of a stage at
// position L ^ (row & 15), L = 8 * plane + p), its sub-block sum and the
// row's 2^-s.
template <int TYPE>
__device__ __forceinline__ void short_prep(const f32x4 (&xv)[8], int tid, KQShortSmem& sm) {
  typedef __attribute__((address_space(3))) u32x4 lds_u32x4_s;
  const int r = tid >> 3, j = tid & 7;
  float v[32];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    v[4 * i] = xv[i].x;
    v[4 * i + 1] = xv[i].y;
    v[4 * i + 2] = xv[i].z;
    v[4 * i + 3] = xv[i].w;
  }
  float bmax = 0.0f;
#pragma unroll
  for (int i = 0; i < 32; ++i) bmax = fmaxf(bmax, fabsf(v[i]));
  float smax = bmax;  // the row's max over the superblock: the 8 lanes of the row
  smax = fmaxf(smax, __shfl_xor(smax, 1));
  smax = fmaxf(smax, __shfl_xor(smax, 2));
  smax = fmaxf(smax, __shfl_xor(smax, 4));
  const int e = headroom_exponent(smax);
  const float up = ldexpf(1.0f, e);
  if (j == 0) sm.rs[r] = ldexpf(1.0f, -e);
  // stage and first piece of the block: Q4_K stage j/2 holds blocks 2g, 2g+1
  // (pieces 0-3, 4-7); Q6_K stage 2h + a holds groups a, a+2 of half h
  constexpr bool kQ6 = TYPE == QK_TYPE_Q6_K;
  const int stage = kQ6 ? 2 * (j >> 2) + (j & 1) : j >> 1;
  const int p0 = kQ6 ? 4 * ((j >> 1) & 1) : 4 * (j & 1);
  uint8_t* row = sm.a[stage] + r * 256;
  float gsum[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const float g[8] = {v[8 * q], v[8 * q + 1], v[8 * q + 2], v[8 * q + 3],
                        v[8 * q + 4], v[8 * q + 5], v[8 * q + 6], v[8 * q + 7]};
    uint32_t hh[4], ll[4];
    q8_scaled_planes(g, bmax, up, hh, ll, gsum[q]);
    *reinterpret_cast<lds_u32x4_s*>((__attribute__((address_space(3))) uint8_t*)(row) +
                                    16 * ((p0 + q) ^ (r & 15))) = u32x4{hh[0], hh[1], hh[2], hh[3]};
    *reinterpret_cast<lds_u32x4_s*>((__attribute__((address_space(3))) uint8_t*)(row) +
                                    16 * ((8 + p0 + q) ^ (r & 15))) = u32x4{ll[0], ll[1], ll[2], ll[3]};
  }
  if constexpr (!kQ6) {
    // the prep kernel's order: each lane's 8 in order, then the quad's DPP sums
    const float t = ((gsum[0] + gsum[1]) + (gsum[2] + gsum[3])) * 0.03125f;
    const _Float16 th = static_cast<_Float16>(t);
    sm.xs[r][j] = th;
    sm.xs[r][8 + j] = static_cast<_Float16>(t - static_cast<float>(th));
  }
}

template <int TYPE>
__device__ __forceinline__ void kq_tile_short(const KQGemmArgs& args, KQShortSmem& sm, int nt, int split,
                                              const uint8_t* wmat, float* ymat, int N) {
  constexpr bool kQ6 = TYPE == QK_TYPE_Q6_K;
  constexpr int B = kQ6 ? kQ6KBytes : kQ4KBytes;
  constexpr int QW = kQ6 ? 2 : 1;
  const int n0 = nt * 128;
  const int M = args.M, K = args.K, S = args.S;
  const int sb0 = split * S / args.splits, sb1 = (split + 1) * S / args.splits;
  const int c_last = 4 * sb1 - 1;
  const int tid = static_cast<int>(threadIdx.x);
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = lane >> 5, l32 = lane & 31;

  // this thread's activation block of every superblock (rows past M re-read the last)
  const float* xrow = args.x + static_cast<int64_t>(min(tid >> 3, M - 1)) * K + 32 * (tid & 7);
  auto load_xs = [&](int sb, f32x4 (&xv)[8]) {
#pragma unroll
    for (int i = 0; i < 8; ++i) xv[i] = *reinterpret_cast<const f32x4_a4*>(xrow + 256 * sb + 4 * i);
  };
  const uint8_t* wrow = wmat + static_cast<int64_t>(min(n0 + wave * 32 + l32, N - 1)) * S * B;
  auto load_head = [&](int sb, u32x4& hd, uint32_t& dd) {
    const uint8_t* p = wrow + sb * B;
    if constexpr (kQ6) {
      hd = load16_a2(p + 192);
      dd = load_u16(p + 208);
    } else {
      hd = load16(p);
      dd = 0;
    }
  };
  auto load_q = [&](int c, u32x4 (&q)[QW]) {
    const int g = c & 3;
    const uint8_t* p = wrow + (c >> 2) * B;
    if constexpr (kQ6) {
      q[0] = load16_a2(p + 64 * (g >> 1) + 32 * (g & 1) + 16 * h);
      q[1] = load16_a2(p + 128 + 32 * (g >> 1) + 16 * h);
    } else {
      q[0] = load16(p + 16 + 32 * g + 16 * h);
    }
  };

  f32x16 acc, ph;
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = ph[r] = 0.0f;
  u32x4 wh[2], bq[2][QW];
  uint32_t wd[2];
  f32x4 xv[8];
  load_xs(sb0, xv);
  load_head(sb0, wh[0], wd[0]);
  load_q(4 * sb0, bq[0]);

  typedef __attribute__((address_space(3))) uint8_t lds_b;
  typedef __attribute__((address_space(3))) half8 lds_h8;
  typedef __attribute__((address_space(3))) f32x4 lds_f4;
  const int swz = l32 & 15;
  auto superblock = [&](int sb, const u32x4& hcur, uint32_t dcur, u32x4& hnext, uint32_t& dnext) {
    __syncthreads();  // every wave is past the previous superblock's stages and fold
    short_prep<TYPE>(xv, tid, sm);
    load_xs(min(sb + 1, sb1 - 1), xv);  // the next superblock's, in flight during the stages
    __syncthreads();
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int c = 4 * sb + g;
      load_q(min(c + 1, c_last), bq[(g + 1) & 1]);
      if (g == 2) load_head(min(sb + 1, sb1 - 1), hnext, dnext);
      __builtin_amdgcn_sched_barrier(0);
      half2v cm[2], ce[2];
      if constexpr (kQ6) {
#pragma unroll
        for (int U = 0; U < 2; ++U) {
          const int scv = __builtin_amdgcn_sbfe(static_cast<int>(hcur[2 * (g >> 1) + U]), 8 * (2 * (g & 1)) + 8 * h, 8);
          const _Float16 sh = static_cast<_Float16>(static_cast<int16_t>(scv));
          cm[U] = half2v{sh, sh};
        }
      } else {
        int sc0, mn0, sc1, mn1;
        scale_min_k4(2 * g, hcur.y, hcur.z, hcur.w, sc0, mn0);
        scale_min_k4(2 * g + 1, hcur.y, hcur.z, hcur.w, sc1, mn1);
        const _Float16 s0 = static_cast<_Float16>(static_cast<uint16_t>(sc0));
        const _Float16 s1 = static_cast<_Float16>(static_cast<uint16_t>(sc1));
        cm[0] = half2v{s0, s0};
        ce[0] = cm[0] * half2v{-1024.0f16, -1024.0f16};
        const half2v t1{s1, s1};
        cm[1] = t1 * half2v{0.0625f16, 0.0625f16};
        ce[1] = t1 * half2v{-64.0f16, -64.0f16};
        (void)mn0;
        (void)mn1;
      }
      const lds_b* a_row = (const lds_b*)(sm.a[g]) + l32 * 256;
      auto read_a = [&](int step, half8& ah, half8& al) {
        const int p = 4 * (step >> 1) + 2 * h + (step & 1);
        ah = *reinterpret_cast<const lds_h8*>(a_row + 16 * (p ^ swz));
        al = *reinterpret_cast<const lds_h8*>(a_row + 16 * ((8 + p) ^ swz));
      };
      auto convert = [&](int step, half8& bw, half8& bx) {
        const int U = step >> 1, s2 = step & 1;
        const u32x4 q = bq[g & 1][0];
        if constexpr (kQ6) {
          const u32x4 qh = bq[g & 1][QW - 1];
          if (U)
            weights_q6k<1>(q[2 * s2], q[2 * s2 + 1], qh[2 * s2], qh[2 * s2 + 1], 2 * (g & 1) + 4, cm[1], bw, bx);
          else
            weights_q6k<0>(q[2 * s2], q[2 * s2 + 1], qh[2 * s2], qh[2 * s2 + 1], 2 * (g & 1), cm[0], bw, bx);
        } else {
          bw = U ? weights_fp16<1>(q[2 * s2], q[2 * s2 + 1], cm[1], ce[1])
                 : weights_fp16<0>(q[2 * s2], q[2 * s2 + 1], cm[0], ce[0]);
          bx = bw;
        }
      };
      half8 ah[2], al[2], bw[2], bx[2];
      read_a(0, ah[0], al[0]);
      read_a(1, ah[1], al[1]);
      convert(0, bw[0], bx[0]);
#pragma unroll
      for (int step = 0; step < 4; ++step) {
        const int ab = step & 1;
        ph = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[ab], bw[ab], ph, 0, 0, 0);
        ph = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[ab], bw[ab], ph, 0, 0, 0);
        if constexpr (kQ6) ph = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[ab], bx[ab], ph, 0, 0, 0);
        if (step < 3) convert(step + 1, bw[(step + 1) & 1], bx[(step + 1) & 1]);
        if (step + 2 < 4) read_a(step + 2, ah[ab], al[ab]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    // superblock end: acc += (d 2^-s(m)) * part (Q4_K: - (32 dmin 2^-s(m)) * (X . m))
    float rsr[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const f32x4 t = *reinterpret_cast<const lds_f4*>((const lds_b*)(sm.rs) + 4 * (8 * i + 4 * h));
      rsr[4 * i] = t.x;
      rsr[4 * i + 1] = t.y;
      rsr[4 * i + 2] = t.z;
      rsr[4 * i + 3] = t.w;
    }
    if constexpr (kQ6) {
      const float d = half_bits_to_float(dcur);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        acc[r] = fmaf(d * rsr[r], ph[r], acc[r]);
        ph[r] = 0.0f;
      }
    } else {
      const float dd = half_bits_to_float(hcur.x & 0xFFFFu);
      const float dm = -32.0f * half_bits_to_float(hcur.x >> 16);
      u32x4 min_b;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        int sa, ma, sb2, mb;
        scale_min_k4(2 * q, hcur.y, hcur.z, hcur.w, sa, ma);
        scale_min_k4(2 * q + 1, hcur.y, hcur.z, hcur.w, sb2, mb);
        const half2v mm{static_cast<_Float16>(static_cast<uint16_t>(ma)), static_cast<_Float16>(static_cast<uint16_t>(mb))};
        min_b[q] = __builtin_bit_cast(uint32_t, mm);
      }
      const u32x4 xa = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(
          (const lds_b*)(&sm.xs[0][0]) + 32 * l32 + 16 * h);
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[r] = fmaf(dd * rsr[r], ph[r], acc[r]);
      f32x16 zero;
#pragma unroll
      for (int r = 0; r < 16; ++r) zero[r] = 0.0f;
      ph = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, xa), __builtin_bit_cast(half8, min_b), zero,
                                                  0, 0, 0);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        acc[r] = fmaf(dm * rsr[r], ph[r], acc[r]);
        ph[r] = 0.0f;
      }
    }
  };
  for (int sb = sb0; sb < sb1; sb += 2) {
    superblock(sb, wh[0], wd[0], wh[1], wd[1]);
    if (sb + 1 < sb1) superblock(sb + 1, wh[1], wd[1], wh[0], wd[0]);
  }

  // epilogue: y (the scales are in acc already), or the partial of this split
  float* const part = args.part + static_cast<int64_t>(split) * M * N;
  const int n = n0 + wave * 32 + l32;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int m = 8 * (r >> 2) + 4 * h + (r & 3);
    if (m >= M || n >= N) continue;
    if (args.splits == 1)
      ymat[static_cast<int64_t>(m) * N + n] = acc[r];
    else
      part[static_cast<int64_t>(m) * N + n] = acc[r];
  }
}

// The short-prompt GEMM: grid, work units and matrices as gemm_kq_kernel's
// (one row of 32 x 128 tiles).
template <int TYPE>
__global__ __launch_bounds__(64 * kWaves, 3) void gemm_kq_short_kernel(const KQGemmArgs args) {
  __shared__ __align__(16) KQShortSmem sm;
  const int b = static_cast<int>(blockIdx.x);
  const int u = (b & 7) * args.per_xcd + (b >> 3);
  if ((b >> 3) >= args.per_xcd || u >= args.tiles * args.splits) return;
  const int nt = u / args.splits, split = u % args.splits;
  const int nseg = args.nseg;
  const int j = (nseg > 1 && nt >= args.tile0[1]) + (nseg > 2 && nt >= args.tile0[2]) +
                (nseg > 3 && nt >= args.tile0[3]);
  auto pick = [j](auto f0, auto f1, auto f2, auto f3) {
    return j == 0 ? f0 : j == 1 ? f1 : j == 2 ? f2 : f3;
  };
  const uint8_t* wmat = pick(args.w[0], args.w[1], args.w[2], args.w[3]);
  float* ymat = pick(args.y[0], args.y[1], args.y[2], args.y[3]);
  const int N = pick(args.N[0], args.N[1], args.N[2], args.N[3]);
  const int nt_local = nt - pick(args.tile0[0], args.tile0[1], args.tile0[2], args.tile0[3]);
  if constexpr (TYPE != 0) {
    kq_tile_short<TYPE>(args, sm, nt_local, split, wmat, ymat, N);
  } else {
    if (pick(args.type[0], args.type[1], args.type[2], args.type[3]) == QK_TYPE_Q4_K)
      kq_tile_short<QK_TYPE_Q4_K>(args, sm, nt_local, split, wmat, ymat, N);
    else
      kq_tile_short<QK_TYPE_Q6_K>(args, sm, nt_local, split, wmat, ymat, N);
  }
}

// TYPE: the weight type of every matrix of the launch, or 0 for matrices of
// both types (each workgroup takes its matrix's). Register budget: three
// workgroups per CU (168 VGPRs) except the Q6_K kernels, whose 64-row tile
// needs more (two per CU). At TM = 2 the Q4_K kernel fits 168 with 3 dwords
// spilled (epilogue values, stored before the superblock loop and reloaded
// after it): ffn_gate at M = 512, 608 tiles, then runs as one round instead
// of 512 tiles plus a 96-tile round.
template <int TYPE, int TM, int TN>
__global__ __launch_bounds__(64 * kWaves, TYPE == QK_TYPE_Q6_K ? 2 : 3) void gemm_kq_kernel(const KQGemmArgs args) {
  using C = KQCfg<TM, TN>;
  __shared__ __align__(16) uint8_t slots[2][C::SLOT];
  const int b = static_cast<int>(blockIdx.x);
  // Consecutive tiles go to one XCD (workgroups are dealt to the 8 XCDs in
  // turn) and run along N first, so an XCD keeps one activation tile in its
  // L2 while the weight tiles stream past it.
  // Work unit u = tile * splits + split: split covers superblocks
  // [sb0, sb1) of K (splits > 1 when the tiles alone leave CUs idle).
  const int u = (b & 7) * args.per_xcd + (b >> 3);
  if ((b >> 3) >= args.per_xcd || u >= args.tiles * args.splits) return;
  const int t = u / args.splits, split = u % args.splits;
  const int mt = t / args.n_tiles;
  const int nt = t % args.n_tiles;
  // the n-tile's matrix, field by field (a struct picked by a runtime index
  // would be copied to scratch memory)
  const int nseg = args.nseg;
  const int j = (nseg > 1 && nt >= args.tile0[1]) + (nseg > 2 && nt >= args.tile0[2]) +
                (nseg > 3 && nt >= args.tile0[3]);
  auto pick = [j](auto f0, auto f1, auto f2, auto f3) {
    return j == 0 ? f0 : j == 1 ? f1 : j == 2 ? f2 : f3;
  };
  const uint8_t* wmat = pick(args.w[0], args.w[1], args.w[2], args.w[3]);
  float* ymat = pick(args.y[0], args.y[1], args.y[2], args.y[3]);
  const int N = pick(args.N[0], args.N[1], args.N[2], args.N[3]);
  const int nt_local = nt - pick(args.tile0[0], args.tile0[1], args.tile0[2], args.tile0[3]);
  if constexpr (TYPE != 0) {
    kq_tile<TYPE, TM, TN>(args, slots, mt, nt_local, split, wmat, ymat, N);
  } else {
    if (pick(args.type[0], args.type[1], args.type[2], args.type[3]) == QK_TYPE_Q4_K)
      kq_tile<QK_TYPE_Q4_K, TM, TN>(args, slots, mt, nt_local, split, wmat, ymat, N);
    else
      kq_tile<QK_TYPE_Q6_K, TM, TN>(args, slots, mt, nt_local, split, wmat, ymat, N);
  }
}

// y[m][n] = (partial 0 + partial 1 + ...) * 2^-s(m) (row_scale null: the
// short-prompt GEMM's partials carry their scales), the splits added in
// order (results do not depend on timing). Grid (ceil(N / 256), M). The
// partials were written on every XCD and miss this one's L2, so each thread
// has 16 splits' loads in flight at once (indices past the last re-read it)
// instead of one load per dependent add.
__global__ __launch_bounds__(256) void gemm_kq_reduce_kernel(const float* __restrict__ part,
                                                             const float* __restrict__ row_scale,
                                                             float* __restrict__ y, int M, int N,
                                                             int splits) {
  constexpr int kBatch = 16;
  const int m = static_cast<int>(blockIdx.y);
  const int n = static_cast<int>(blockIdx.x) * 256 + static_cast<int>(threadIdx.x);
  if (n >= N) return;
  const int64_t at = static_cast<int64_t>(m) * N + n, plane = static_cast<int64_t>(M) * N;
  float v = 0.0f;
  for (int k0 = 0; k0 < splits; k0 += kBatch) {
    float p[kBatch];
#pragma unroll
    for (int kk = 0; kk < kBatch; ++kk) p[kk] = part[min(k0 + kk, splits - 1) * plane + at];
#pragma unroll
    for (int kk = 0; kk < kBatch; ++kk)
      if (k0 + kk < splits) v = k0 + kk == 0 ? p[kk] : v + p[kk];
  }
  y[at] = row_scale ? v * row_scale[m] : v;
}

template <int TYPE, int TM, int TN>
hipError_t launch_cfg(KQGemmArgs a, hipStream_t stream) {
  using C = KQCfg<TM, TN>;
  a.n_tiles = 0;
  for (int j = 0; j < a.nseg; ++j) {
    a.tile0[j] = a.n_tiles;
    a.n_tiles += (a.N[j] + C::BN - 1) / C::BN;
  }
  a.tiles = a.n_tiles * ((a.M + C::BM - 1) / C::BM);
  a.per_xcd = (a.tiles * a.splits + 7) / 8;
  note("gemm_kq_kernel", 8 * a.per_xcd, TYPE, TM, TN, a.splits);
  hipLaunchKernelGGL((gemm_kq_kernel<TYPE, TM, TN>), dim3(static_cast<uint32_t>(8 * a.per_xcd)),
                     dim3(64 * kWaves), 0, stream, a);
  return hipGetLastError();
}

template <int TYPE>
hipError_t launch_short(KQGemmArgs a, hipStream_t stream) {
  a.n_tiles = 0;
  for (int j = 0; j < a.nseg; ++j) {
    a.tile0[j] = a.n_tiles;
    a.n_tiles += (a.N[j] + 127) / 128;
  }
  a.tiles = a.n_tiles;  // one row of tiles
  a.per_xcd = (a.tiles * a.splits + 7) / 8;
  note("gemm_kq_short_kernel", 8 * a.per_xcd, TYPE, a.splits);
  hipLaunchKernelGGL((gemm_kq_short_kernel<TYPE>), dim3(static_cast<uint32_t>(8 * a.per_xcd)), dim3(64 * kWaves), 0,
                     stream, a);
  return hipGetLastError();
}

struct KQPlan {
  bool wide;   // 64 x 128 tiles, else 32 x 128
  int splits;  // K split into this many superblock ranges
};

// Tile and split choice, planned for MI355X's 256 CUs (correct on any
// device): 64 x 128 tiles when the grid is large enough, else 32 x 128
// (twice the workgroups, each half the rows). Q4_K takes 64 x 128 from 1.5
// tiles per CU (measured, N = 9728: M = 384, 456 tiles, 65.7 us against 75.7
// with 912 narrow tiles; M = 320, 380 tiles, no difference) and 32 x 128
// below (attn_q/k, attn_output at M = 512); Q6_K, whose stages cost more,
// takes 64 x 128 from half a tile per CU (ffn_down) and 32 x 128 below
// (attn_v). The tile height does not change any output element's sums. Grids of fewer than two
// tiles per CU split K (at most 4 ways, at least 4 superblocks a split) so
// that about two work units reach every CU; a reduce kernel adds the splits.
// Measured at M = 512: ffn_down (K = 9728, 3 splits) 102 us with its reduce
// against 137; attn_k / attn_v alone (K = 2560, 128 tiles, 2 splits of 5
// superblocks) 26.3 -> 22.4 us and 33.3 -> 27.1 us.
// At M <= 32 (one row of tiles: a short prompt) K splits down to single
// superblocks. Measured at M = 23 (graph replays over 36 distinct layers,
// prep and reduce included): ffn_gate 27.1 -> 20.8 us, attn_k 23.1 -> 12.7,
// ffn_down 41.3 -> 36.2.
constexpr int64_t kPlanCUs = 256;

KQPlan plan(int type, int64_t M, int64_t N, int64_t K) {
  const int64_t tiles64 = ((M + 63) / 64) * ((N + 127) / 128);
  const int64_t tiles32 = ((M + 31) / 32) * ((N + 127) / 128);
  // (M <= 32: one row of tiles either way, and a 64-row tile would compute
  // its padding rows: the lm_head at M = 23 is 1187 tiles of either height)
  const bool wide = M > 32 && (type == QK_TYPE_Q6_K ? 2 * tiles64 >= kPlanCUs : 2 * tiles64 >= 3 * kPlanCUs);
  const int64_t tiles = wide ? tiles64 : tiles32;
  // One row of 32-row tiles (a short prompt): every work unit would walk all
  // of K at ~0.7 us a 64-weight stage, so K splits down to one superblock per
  // unit until about two units reach every CU (the partial products are
  // small at this M).
  const bool short_m = M <= 32;
  const int64_t by_grid = short_m ? std::clamp<int64_t>((2 * kPlanCUs + tiles - 1) / tiles, 1, K / 256)
                                  : std::clamp<int64_t>(2 * kPlanCUs / tiles, 1, 4);
  const int64_t by_depth = short_m ? K / 256 : std::max<int64_t>(K / 256 / 4, 1);
  // (fewer than 512 tiles also keeps M below 16384, inside the reduce grid's
  // 65535 rows; the check states it)
  const bool fits_reduce = M <= 65535;
  return {wide, fits_reduce ? static_cast<int>(std::min(by_grid, by_depth)) : 1};
}

}  // namespace

bool gemm_kq_fits(int64_t M, int64_t K, int64_t N) {
  return K % 256 == 0 && M > 0 && N > 0 && M <= (1 << 30) && N <= (1 << 30) &&
         M * N <= (int64_t{1} << 40);
}

size_t gemm_kq_partial_bytes(int type, int64_t M, int64_t K, int64_t N) {
  const KQPlan p = plan(type, M, N, K);
  return p.splits > 1 ? static_cast<size_t>(p.splits) * M * N * sizeof(float) : 0;
}

hipError_t launch_gemm_kq(int type, const float* x, const _Float16* hi, const float* row_scale,
                          const void* xsums, const void* w, int64_t K, int64_t N, float* y, int64_t M,
                          float* partials, hipStream_t stream) {
  const KQPlan p = plan(type, M, N, K);
  const bool short_m = x != nullptr;  // the short form: planes formed from x in the GEMM
  if (short_m && M > kShortM) return hipErrorInvalidValue;
  KQGemmArgs a{};
  a.x = x;
  a.hi = hi;
  a.xs = static_cast<const _Float16*>(xsums);
  a.row_scale = row_scale;
  a.nseg = 1;
  a.w[0] = static_cast<const uint8_t*>(w);
  a.y[0] = y;
  a.N[0] = static_cast<int32_t>(N);
  a.type[0] = type;
  a.part = partials;
  a.M = static_cast<int32_t>(M);
  a.K = static_cast<int32_t>(K);
  a.S = static_cast<int32_t>(K / 256);
  a.splits = p.splits;
  if (p.splits > 1 && partials == nullptr) return hipErrorInvalidValue;
  hipError_t e;
  if (short_m)
    e = type == QK_TYPE_Q6_K ? launch_short<QK_TYPE_Q6_K>(a, stream) : launch_short<QK_TYPE_Q4_K>(a, stream);
  else if (type == QK_TYPE_Q6_K)
    e = p.wide ? launch_cfg<QK_TYPE_Q6_K, 2, 1>(a, stream) : launch_cfg<QK_TYPE_Q6_K, 1, 1>(a, stream);
  else
    e = p.wide ? launch_cfg<QK_TYPE_Q4_K, 2, 1>(a, stream) : launch_cfg<QK_TYPE_Q4_K, 1, 1>(a, stream);
  if (e != hipSuccess || p.splits == 1) return e;
  gemm_kq_reduce_kernel<<<dim3(static_cast<uint32_t>((N + 255) / 256), static_cast<uint32_t>(M)), 256,
                          0, stream>>>(partials, short_m ? nullptr : row_scale, y, static_cast<int>(M),
                                       static_cast<int>(N), p.splits);
  return hipGetLastError();
}

hipError_t launch_gemm_kq_multi(const float* x, const _Float16* hi, const float* row_scale, const void* xsums,
                                const qk_segment* segments, int count, int64_t K, int64_t M,
                                hipStream_t stream, bool& launched) {
  launched = false;
  if (count < 2 || count > kKQMaxSegments) return hipSuccess;
  // One launch when the combined grid needs no split of K: each tile then
  // does exactly the work of an unsplit launch of its matrix (outputs bit for
  // bit those of the single launch when that does not split; within the
  // splits' rounding of it otherwise: a split changes the order of the sums),
  // in one grid that fills the CUs. Q6_K matrices first: their tiles take
  // longer, so they start first.
  int order[kKQMaxSegments], n = 0;
  bool q4 = false, q6 = false;
  int64_t total = 0;
  for (int pass = 0; pass < 2; ++pass)
    for (int j = 0; j < count; ++j)
      if ((segments[j].type == QK_TYPE_Q6_K) == (pass == 0)) order[n++] = j;
  for (int j = 0; j < count; ++j) {
    if (!gemm_kq_fits(M, K, segments[j].N)) return hipSuccess;
    (segments[j].type == QK_TYPE_Q4_K ? q4 : q6) = true;
    total += segments[j].N;
  }
  if (!gemm_kq_fits(M, K, total)) return hipSuccess;
  const int type = q4 && q6 ? 0 : q4 ? QK_TYPE_Q4_K : QK_TYPE_Q6_K;
  if (plan(type == 0 ? QK_TYPE_Q4_K : type, M, total, K).splits > 1) return hipSuccess;
  // The tile shape of the combined grid. The mixed-type kernel exists for
  // 32 x 128 tiles only: it is taken while the grid has fewer than two
  // 64 x 128 tiles per CU (q + k + v at M = 512: 384), else same-type pairs run.
  const bool short_m = x != nullptr;
  if (short_m && M > kShortM) return hipErrorInvalidValue;
  bool wide = false;
  if (type == 0 && !short_m) {
    if (((M + 63) / 64) * ((total + 127) / 128) >= 2 * kPlanCUs) return hipSuccess;
  } else if (type != 0) {
    wide = plan(type, M, total, K).wide;
  }
  KQGemmArgs a{};
  a.x = x;
  a.hi = hi;
  a.xs = static_cast<const _Float16*>(xsums);
  a.row_scale = row_scale;
  a.nseg = count;
  for (int i = 0; i < count; ++i) {
    const qk_segment& sg = segments[order[i]];
    a.w[i] = static_cast<const uint8_t*>(sg.w);
    a.y[i] = sg.y;
    a.N[i] = static_cast<int32_t>(sg.N);
    a.type[i] = sg.type;
  }
  a.M = static_cast<int32_t>(M);
  a.K = static_cast<int32_t>(K);
  a.S = static_cast<int32_t>(K / 256);
  a.splits = 1;
  hipError_t e;
  if (short_m)
    e = type == 0 ? launch_short<0>(a, stream)
                  : type == QK_TYPE_Q6_K ? launch_short<QK_TYPE_Q6_K>(a, stream) : launch_short<QK_TYPE_Q4_K>(a, stream);
  else if (type == 0)
    e = launch_cfg<0, 1, 1>(a, stream);
  else if (type == QK_TYPE_Q6_K)
    e = wide ? launch_cfg<QK_TYPE_Q6_K, 2, 1>(a, stream) : launch_cfg<QK_TYPE_Q6_K, 1, 1>(a, stream);
  else
    e = wide ? launch_cfg<QK_TYPE_Q4_K, 2, 1>(a, stream) : launch_cfg<QK_TYPE_Q4_K, 1, 1>(a, stream);
  launched = e == hipSuccess;
  return e;
}

}  // namespace qk
