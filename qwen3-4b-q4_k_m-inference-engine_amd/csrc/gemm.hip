// Q4_K / Q6_K dequantize-GEMM for prefill (M > 8 activation rows), on MFMA.
//
// Replaces project<T> launched with gridDim.y = rows (src/cuda/matmul.cu:151-158),
// which re-reads the whole weight matrix once per activation row. Here:
//   1. prep_rows_kernel: per activation row, the Q8 round trip of x
//      (MatmulReference.hpp:11-29: round(x/amax*127) * (amax/127) per 32
//      values), scaled by a power of two 2^s that brings the row's largest
//      |x| into [2^14, 2^15), then split into two fp16 planes hi + lo with
//      hi = fp16(v), lo = fp16(v - hi): 22 significant bits of v.
//   2. gemm_kernel: 128 x BN output tiles, 8 waves: two K groups of 4 waves
//      of 64 x BN/2 (alternate 16-deep steps, summed through LDS at the end),
//      each a grid of v_mfma_f32_32x32x16_f16 tiles with fp32 accumulators,
//      tiles dealt XCD by XCD so a weight tile stays in one L2. Per K-chunk
//      of 32 weights (one scale group) the workgroup dequantises BN weight
//      rows straight from the GGUF superblocks with the fp32 formula of
//      src/cuda/embedding.cu:6-59, scaled by a per-row power of two 2^t
//      (found from the row's superblock headers so the row's |w| bound lands
//      in [2^14, 2^15)), split into fp16 hi + lo, into LDS beside the
//      activation tile. Each 16-deep step issues hi*hi + hi*lo + lo*hi, which
//      leaves an operand error near 2^-22 relative: the products carry about
//      the precision of the fp32 reference path, not that of fp16.
//      Epilogue: y = acc * 2^-s(m) * 2^-t(n) (exact scalings).
//   Chunks are double buffered in LDS and their global loads run two chunks
//   ahead in registers.
// MFMA operand rule (checked on the device): lane l gives row l%32 of A and
// column l%32 of B with the same 8 k values, half-wave l/32 choosing which 8;
// D lane l, register r holds row 8*(r/4) + 4*(l/32) + r%4, column l%32.
#include "qk_device.hpp"
#include "qk_launch.hpp"

namespace qk {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));

constexpr int kBM = 128;                  // activation rows per tile
constexpr int kBK = 32;                   // weights per K-chunk (one scale group)
constexpr int kRowBytes = 2 * kBK * 2 + 16;  // LDS row: hi[32], lo[32] halves, 16 B pad
constexpr int kHeadroomExp = 14;          // scaled magnitudes below 2^15 < fp16 max

// Power-of-two exponent that brings a positive finite bound into
// [2^14, 2^15); 0 for 0, clamped for inf/nan bounds (their products are
// inf/nan whatever the scale).
__device__ __forceinline__ int headroom_exponent(float bound) {
  if (!(bound > 0.0f)) return 0;
  if (!(bound <= 3.0e38f)) return -64;
  return min(kHeadroomExp - ilogbf(bound), 100);  // 2^s and 2^-s stay normal floats
}

__device__ __forceinline__ uint32_t pack2(float a, float b) {
  return __builtin_bit_cast(uint32_t, half2v{static_cast<_Float16>(a), static_cast<_Float16>(b)});
}

// v -> (fp16(v), fp16(v - fp16(v))) for a pair of values, packed.
__device__ __forceinline__ void split2(float a, float b, uint32_t& hi, uint32_t& lo) {
  const _Float16 ha = static_cast<_Float16>(a), hb = static_cast<_Float16>(b);
  hi = __builtin_bit_cast(uint32_t, half2v{ha, hb});
  lo = pack2(a - static_cast<float>(ha), b - static_cast<float>(hb));
}

// ---------------------------------------------------------------- prep ------

// Q8 round trip of one group of 8 activations (a quad of lanes holds one
// 32-value block), scaled by `up`, split into fp16 hi/lo at hi + at, lo + at.
// The quad's first lane also stores 2^-5 * (sum of the block's scaled
// values) as hi/lo at xs + xs_at (the Q4_K GEMM's min-term operand).
__device__ __forceinline__ void prep_group(const f32x4 a, const f32x4 b, float up,
                                           _Float16* __restrict__ hi, _Float16* __restrict__ lo,
                                           int64_t at, _Float16* __restrict__ xs, int64_t xs_at,
                                           bool first) {
  const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  float bmax = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) bmax = fmaxf(bmax, fabsf(v[i]));
  bmax = fmaxf(bmax, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                         0, __builtin_bit_cast(int, bmax), 0xB1, 0xF, 0xF, false)));
  bmax = fmaxf(bmax, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                         0, __builtin_bit_cast(int, bmax), 0x4E, 0xF, 0xF, false)));
  const float scale = bmax / 127.0f;
  uint32_t h[4], l[4];
  float sum = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float c0 = bmax == 0.0f ? 0.0f : roundf((v[2 * i] / bmax) * 127.0f);
    const float c1 = bmax == 0.0f ? 0.0f : roundf((v[2 * i + 1] / bmax) * 127.0f);
    const float s0 = (c0 * scale) * up, s1 = (c1 * scale) * up;
    split2(s0, s1, h[i], l[i]);
    sum += s0;
    sum += s1;
  }
  *reinterpret_cast<u32x4*>(hi + at) = u32x4{h[0], h[1], h[2], h[3]};
  *reinterpret_cast<u32x4*>(lo + at) = u32x4{l[0], l[1], l[2], l[3]};
  sum += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, sum), 0xB1,
                                                               0xF, 0xF, false));
  sum += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, sum), 0x4E,
                                                               0xF, 0xF, false));
  if (first) {
    const float t = sum * 0.03125f;
    const _Float16 th = static_cast<_Float16>(t);
    xs[xs_at] = th;
    xs[xs_at + 8] = static_cast<_Float16>(t - static_cast<float>(th));
  }
}

// Sub-block sums layout: 32 bytes per (row, superblock of 256 values): the
// 8 hi halves, then the 8 lo halves. Index (in halves) of block jb's hi value.
__device__ __forceinline__ int64_t xsum_index(int64_t row, int jb, int S) {
  return (row * S + (jb >> 3)) * 16 + (jb & 7);
}

constexpr int kPrepGroups = 8;  // groups of 8 activations held per thread: K <= 16384 in one pass

// One workgroup per activation row: the row's max |x| (for the power-of-two
// scale), then the Q8 round trip of every 32-value block. Rows up to 16384
// values stay in registers between the two steps; wider rows are read twice.
// K % 32 == 0, so the 4 lanes of a quad are always in or out together.
__global__ __launch_bounds__(256) void prep_rows_kernel(const float* __restrict__ x,
                                                        _Float16* __restrict__ hi,
                                                        _Float16* __restrict__ lo,
                                                        float* __restrict__ row_scale,
                                                        _Float16* __restrict__ xs, int K) {
  __shared__ float partial[4];
  const int64_t row = blockIdx.x;
  const float* xr = x + row * K;
  const int tid = static_cast<int>(threadIdx.x);
  const int groups = K / 8;
  const bool resident = groups <= 256 * kPrepGroups;
  f32x4 va[kPrepGroups], vb[kPrepGroups];
  float amax = 0.0f;
  if (resident) {
#pragma unroll
    for (int i = 0; i < kPrepGroups; ++i) {
      const int g = tid + 256 * i;
      va[i] = vb[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      if (g < groups) {
        va[i] = *reinterpret_cast<const f32x4_a4*>(xr + 8 * g);
        vb[i] = *reinterpret_cast<const f32x4_a4*>(xr + 8 * g + 4);
      }
      const f32x4 m4 = f32x4{fmaxf(fabsf(va[i].x), fabsf(vb[i].x)), fmaxf(fabsf(va[i].y), fabsf(vb[i].y)),
                             fmaxf(fabsf(va[i].z), fabsf(vb[i].z)), fmaxf(fabsf(va[i].w), fabsf(vb[i].w))};
      amax = fmaxf(amax, fmaxf(fmaxf(m4.x, m4.y), fmaxf(m4.z, m4.w)));
    }
  } else {
    for (int i = 4 * tid; i < K; i += 1024) {
      const f32x4 v = *reinterpret_cast<const f32x4_a4*>(xr + i);
      amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    }
  }
  for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
  if ((tid & 63) == 0) partial[tid >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(partial[0], partial[1]), fmaxf(partial[2], partial[3]));
  const int s = headroom_exponent(amax);
  const float up = ldexpf(1.0f, s);
  if (tid == 0) row_scale[row] = ldexpf(1.0f, -s);

  if (resident) {
#pragma unroll
    for (int i = 0; i < kPrepGroups; ++i) {
      const int g = tid + 256 * i;
      if (g < groups)
        prep_group(va[i], vb[i], up, hi, lo, row * K + 8 * g, xs, xsum_index(row, g >> 2, K / 256),
                   (g & 3) == 0);
    }
  } else {
    for (int g = tid; g < groups; g += 256)
      prep_group(*reinterpret_cast<const f32x4_a4*>(xr + 8 * g),
                 *reinterpret_cast<const f32x4_a4*>(xr + 8 * g + 4), up, hi, lo, row * K + 8 * g,
                 xs, xsum_index(row, g >> 2, K / 256), (g & 3) == 0);
  }
}

// ------------------------------------------------------- weight staging -----

// Raw bytes one thread needs for its BPT weights of one K-chunk (scale group
// j = kc % 8 of superblock kc / 8) of one weight row.
template <int TYPE, int BPT>
struct RawW;

template <int BPT>
struct RawW<QK_TYPE_Q4_K, BPT> {
  u32x4 head;  // d, dmin, scales[12]
  uint32_t qs[BPT / 4];
};

template <int BPT>
struct RawW<QK_TYPE_Q6_K, BPT> {
  uint32_t ql[BPT / 4 + 1], qh[BPT / 4 + 1];  // from the dword at or below the field
  int32_t sc;                                  // int8 scale of this part's 16-weight half
  uint32_t d_bits, shift;                      // d; field misalignment in bits (0 or 16)
};

// Group j of a Q4_K superblock: the low (j even) or high nibbles of qs bytes
// 32*(j/2) .. +31; this part's weights l = p*BPT .. +BPT-1 of the group.
template <int BPT>
__device__ __forceinline__ void load_raw(const uint8_t* wrow, int kc, int p,
                                         RawW<QK_TYPE_Q4_K, BPT>& r) {
  const uint8_t* sb = wrow + (kc >> 3) * kQ4KBytes;
  r.head = load16(sb);
  const uint8_t* qs = sb + 16 + 32 * ((kc & 7) >> 1) + p * BPT;
#pragma unroll
  for (int i = 0; i < BPT / 4; ++i) r.qs[i] = load_u32(qs + 4 * i);
}

// Group j of a Q6_K superblock: half h = j/4, g = j%4 (src/cuda/embedding.cu:41-57):
// low bits from ql[64h + 32(g&1) + l] (nibble g/2), high bits 2g..2g+1 of
// qh[32h + l], scale scales[8h + 2g + l/16].
template <int BPT>
__device__ __forceinline__ void load_raw(const uint8_t* wrow, int kc, int p,
                                         RawW<QK_TYPE_Q6_K, BPT>& r) {
  const uint8_t* sb = wrow + (kc >> 3) * kQ6KBytes;
  const uint32_t mis = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(sb)) & 3u;
  const uint8_t* base = sb - mis;
  const int j = kc & 7, h = j >> 2, g = j & 3;
  const uint8_t* ql = base + 64 * h + 32 * (g & 1) + p * BPT;
  const uint8_t* qh = base + 128 + 32 * h + p * BPT;
#pragma unroll
  for (int i = 0; i <= BPT / 4; ++i) {
    r.ql[i] = load_u32(ql + 4 * i);
    r.qh[i] = load_u32(qh + 4 * i);
  }
  r.sc = reinterpret_cast<const int8_t*>(sb)[192 + 8 * h + 2 * g + (p * BPT >= 16 ? 1 : 0)];
  r.d_bits = load_u16(sb + 208);
  r.shift = 8 * mis;
}

// Bound on |w| over one superblock from its header, for the row scale.
__device__ __forceinline__ float superblock_bound(const uint8_t* sb, int type) {
  if (type == QK_TYPE_Q4_K) {
    const uint32_t dd = load_u32(sb);
    return 945.0f * fabsf(half_bits_to_float(dd & 0xFFFFu)) +
           63.0f * fabsf(half_bits_to_float(dd >> 16));
  }
  return 4096.0f * fabsf(half_bits_to_float(load_u16(sb + 208)));
}

// Store the part's BPT split weights: hi at lds_row + 2*p*BPT, lo 64 bytes on.
template <int BPT>
__device__ __forceinline__ void store_split(const uint32_t (&hi)[BPT / 2],
                                            const uint32_t (&lo)[BPT / 2], int p,
                                            uint8_t* lds_row) {
  uint8_t* dh = lds_row + 2 * p * BPT;
  uint8_t* dl = dh + 2 * kBK;
  if constexpr (BPT >= 8) {
#pragma unroll
    for (int i = 0; i < BPT / 8; ++i) {
      reinterpret_cast<u32x4*>(dh)[i] = u32x4{hi[4 * i], hi[4 * i + 1], hi[4 * i + 2], hi[4 * i + 3]};
      reinterpret_cast<u32x4*>(dl)[i] = u32x4{lo[4 * i], lo[4 * i + 1], lo[4 * i + 2], lo[4 * i + 3]};
    }
  } else {
    static_assert(BPT == 4, "4 or a multiple of 8 weights per thread");
    *reinterpret_cast<uint2*>(dh) = make_uint2(hi[0], hi[1]);
    *reinterpret_cast<uint2*>(dl) = make_uint2(lo[0], lo[1]);
  }
}

// Byte N of v as a float (one v_cvt_f32_ubyteN).
template <int N>
__device__ __forceinline__ float byte_f(uint32_t v) {
  return static_cast<float>((v >> (8 * N)) & 0xFFu);
}

template <int BPT>
__device__ __forceinline__ void dequant_store(const RawW<QK_TYPE_Q4_K, BPT>& r, int kc, int p,
                                              float ws, uint8_t* lds_row) {
  const uint32_t j = kc & 7;
  int sc, m;
  scale_min_k4(j, r.head.y, r.head.z, r.head.w, sc, m);
  // (d*sc)*q - dmin*m as src/cuda/embedding.cu:24-31, every factor scaled by 2^t (exact)
  const float ds = (half_bits_to_float(r.head.x & 0xFFFFu) * ws) * static_cast<float>(sc);
  const float dm = (half_bits_to_float(r.head.x >> 16) * ws) * static_cast<float>(m);
  const uint32_t nib = 4 * (j & 1);
  uint32_t hi[BPT / 2], lo[BPT / 2];
#pragma unroll
  for (int i = 0; i < BPT / 4; ++i) {
    const uint32_t q = (r.qs[i] >> nib) & 0x0F0F0F0Fu;
    split2(byte_f<0>(q) * ds - dm, byte_f<1>(q) * ds - dm, hi[2 * i], lo[2 * i]);
    split2(byte_f<2>(q) * ds - dm, byte_f<3>(q) * ds - dm, hi[2 * i + 1], lo[2 * i + 1]);
  }
  store_split<BPT>(hi, lo, p, lds_row);
}

template <int BPT>
__device__ __forceinline__ void dequant_store(const RawW<QK_TYPE_Q6_K, BPT>& r, int kc, int p,
                                              float ws, uint8_t* lds_row) {
  const int g = kc & 3;
  const uint32_t nib = 4u * (g >> 1), hsh = 2u * g;
  // d * sc * (q - 32) as src/cuda/embedding.cu:49-55, d scaled by 2^t (exact)
  const float ds = (half_bits_to_float(r.d_bits) * ws) * static_cast<float>(r.sc);
  uint32_t hi[BPT / 2], lo[BPT / 2];
#pragma unroll
  for (int i = 0; i < BPT / 4; ++i) {
    const uint32_t a = __builtin_amdgcn_alignbit(r.ql[i + 1], r.ql[i], r.shift);
    const uint32_t b = __builtin_amdgcn_alignbit(r.qh[i + 1], r.qh[i], r.shift);
    const uint32_t q = ((a >> nib) & 0x0F0F0F0Fu) | (((b >> hsh) & 0x03030303u) << 4);
    split2((byte_f<0>(q) - 32.0f) * ds, (byte_f<1>(q) - 32.0f) * ds, hi[2 * i], lo[2 * i]);
    split2((byte_f<2>(q) - 32.0f) * ds, (byte_f<3>(q) - 32.0f) * ds, hi[2 * i + 1], lo[2 * i + 1]);
  }
  store_split<BPT>(hi, lo, p, lds_row);
}

// ---------------------------------------------------------------- GEMM ------

struct GemmArgs {
  const _Float16* hi;      // [M x K] activation planes
  const _Float16* lo;
  const float* row_scale;  // [M] 2^-s
  const uint8_t* w;
  float* y;
  int M, N, K;
};

constexpr int kGemmWaves = 8;
constexpr int kGemmThreads = 64 * kGemmWaves;

template <int TYPE, int BN>
struct GemmStage {
  static constexpr int kTPR = kGemmThreads / BN;  // threads per weight row
  static constexpr int kBPT = kBK / kTPR;         // weights per thread per chunk
  u32x4 a[2];                                     // 2 x 16 B of the activation planes
  RawW<TYPE, kBPT> w;
};

// Tile t of the launch for workgroup b: consecutive tiles (the m-tiles of one
// weight tile first) go to the same XCD (workgroups are dealt to the 8 XCDs
// round-robin), so a weight tile is fetched into one L2 and reused there.
__device__ __forceinline__ int xcd_tile(int b, int grid) {
  const int per_xcd = grid / 8;  // grid is a multiple of 8
  return (b % 8) * per_xcd + b / 8;
}

// 8 waves: waves 0-3 and 4-7 form two K groups that take alternate 16-deep
// steps of every chunk on the same 128 x BN tile (each wave 64 x BN/2), so
// every SIMD runs two waves; group 1's accumulators are added to group 0's
// through LDS at the end (a fixed order: the result does not depend on timing).
template <int TYPE, int BN>
__global__ __launch_bounds__(kGemmThreads) void gemm_kernel(const GemmArgs args, int tiles) {
  using Stage = GemmStage<TYPE, BN>;
  constexpr int kTPR = Stage::kTPR, kBPT = Stage::kBPT;
  constexpr int kNT = BN / 64;  // 32-wide MFMA tiles per wave along N
  constexpr int kBytes = TYPE == QK_TYPE_Q4_K ? kQ4KBytes : kQ6KBytes;
  constexpr int kStage = (kBM + BN) * kRowBytes;
  static_assert(4 * 64 * 2 * kNT * 16 * 4 <= 2 * kStage, "reduction fits the stage buffers");
  __shared__ __align__(16) uint8_t lds[2 * kStage];
  __shared__ float col_scale[BN];
  __shared__ float row_scale[kBM];

  const int tile = xcd_tile(static_cast<int>(blockIdx.x), static_cast<int>(gridDim.x));
  if (tile >= tiles) return;  // whole workgroup, before any barrier
  const int M = args.M, N = args.N, K = args.K;
  const int tid = static_cast<int>(threadIdx.x);
  const int lane = tid & 63, wave = tid >> 6;
  const int kgroup = wave >> 2, wq = wave & 3;
  const int m_tiles = (M + kBM - 1) / kBM;
  const int m0 = (tile % m_tiles) * kBM;
  const int n0 = (tile / m_tiles) * BN;
  const int wm = (wq & 1) * 64, wn = (wq >> 1) * (BN / 2);
  const int nk = K / kBK;
  const int S = K / 256;

  // activation pieces: 16 B = 8 halves; piece (tid & 7) of a 128-byte LDS row
  // image (hi 0..3, lo 4..7), rows (tid >> 3) + 64 i (clamped; never stored)
  const int a_piece = tid & 7;
  const _Float16* plane = (a_piece < 4 ? args.hi : args.lo) + (a_piece & 3) * 8;
  const _Float16* a_src[2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
    a_src[i] = plane + static_cast<int64_t>(min(m0 + (tid >> 3) + 64 * i, M - 1)) * K;

  const int w_local = tid / kTPR, w_part = tid % kTPR;
  const uint8_t* w_row = args.w + static_cast<int64_t>(min(n0 + w_local, N - 1)) * S * kBytes;

  // per-row weight scale 2^t from the row's superblock headers
  float bound = 0.0f;
  for (int s = w_part; s < S; s += kTPR)
    bound = fmaxf(bound, superblock_bound(w_row + s * kBytes, TYPE));
#pragma unroll
  for (int off = 1; off < kTPR; off <<= 1) bound = fmaxf(bound, __shfl_xor(bound, off));
  const int t = headroom_exponent(bound);
  const float wscale = ldexpf(1.0f, t);
  if (w_part == 0) col_scale[w_local] = ldexpf(1.0f, -t);
  if (tid < kBM) row_scale[tid] = args.row_scale[min(m0 + tid, M - 1)];

  auto load_stage = [&](int kc, Stage& st) {
#pragma unroll
    for (int i = 0; i < 2; ++i) st.a[i] = load16(a_src[i] + kc * kBK);
    load_raw<kBPT>(w_row, kc, w_part, st.w);
  };
  auto store_stage = [&](int kc, const Stage& st, int buf) {
    uint8_t* base = lds + buf * kStage;
#pragma unroll
    for (int i = 0; i < 2; ++i)
      *reinterpret_cast<u32x4*>(base + ((tid >> 3) + 64 * i) * kRowBytes + a_piece * 16) = st.a[i];
    dequant_store<kBPT>(st.w, kc, w_part, wscale, base + (kBM + w_local) * kRowBytes);
  };

  f32x16 acc[2][kNT];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < kNT; ++j) acc[i][j] = f32x16{};

  // this wave's 16-deep step of the chunk (kgroup 0: k 0..15, 1: k 16..31)
  auto mma_chunk = [&](int buf) {
    const uint8_t* base = lds + buf * kStage + kgroup * 32 + 16 * (lane >> 5);
    half8 ah[2], al[2], bh[kNT], bl[kNT];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const uint8_t* r = base + (wm + 32 * i + (lane & 31)) * kRowBytes;
      ah[i] = *reinterpret_cast<const half8*>(r);
      al[i] = *reinterpret_cast<const half8*>(r + 2 * kBK);
    }
#pragma unroll
    for (int j = 0; j < kNT; ++j) {
      const uint8_t* r = base + (kBM + wn + 32 * j + (lane & 31)) * kRowBytes;
      bh[j] = *reinterpret_cast<const half8*>(r);
      bl[j] = *reinterpret_cast<const half8*>(r + 2 * kBK);
    }
    // one product term over every tile before the next term, so each
    // accumulator's dependent MFMAs are 2*kNT issues apart
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < kNT; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[i], bh[j], acc[i][j], 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < kNT; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i], bl[j], acc[i][j], 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < kNT; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i], bh[j], acc[i][j], 0, 0, 0);
  };

  // A ring of kDepth register stages keeps the global loads kDepth-1 chunks
  // ahead of their dequantisation (HBM latency is several chunk times); two
  // LDS buffers alternate. Step c: load chunk c+kDepth into the stage chunk c
  // vacated, multiply chunk c from LDS, dequantise and store chunk c+1 into
  // the other buffer, barrier. Loads past the end re-read the last chunk (in
  // bounds, unused) so no load sits under a branch. nk is a multiple of 8.
  constexpr int kDepth = 4;
  Stage st[kDepth];
#pragma unroll
  for (int i = 0; i < kDepth; ++i) load_stage(i, st[i]);
  store_stage(0, st[0], 0);
  __syncthreads();
  for (int kc = 0; kc < nk; kc += kDepth) {
#pragma unroll
    for (int i = 0; i < kDepth; ++i) {
      const int c = kc + i;
      load_stage(min(c + kDepth, nk - 1), st[i]);
      mma_chunk(i & 1);
      if (c + 1 < nk) store_stage(c + 1, st[(i + 1) % kDepth], (i + 1) & 1);
      __syncthreads();
    }
  }

  // K group 1 hands its partial tile to group 0 (lane-major so the stores and
  // loads of a wave are contiguous)
  float* red = reinterpret_cast<float*>(lds) + wq * (2 * kNT * 16 * 64);
  if (kgroup == 1) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < kNT; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) red[((i * kNT + j) * 16 + r) * 64 + lane] = acc[i][j][r];
  }
  __syncthreads();
  if (kgroup == 1) return;

  // epilogue: D lane l, register r -> row 8*(r/4) + 4*(l/32) + r%4, column l%32
  float* __restrict__ y = args.y;
#pragma unroll
  for (int j = 0; j < kNT; ++j) {
    const int nl = wn + 32 * j + (lane & 31);
    const int n = n0 + nl;
    const float cs = col_scale[nl];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + wm + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        const float v = acc[i][j][r] + red[((i * kNT + j) * 16 + r) * 64 + lane];
        if (m < M && n < N) y[static_cast<int64_t>(m) * N + n] = (v * row_scale[m - m0]) * cs;
      }
  }
}

template <int TYPE>
hipError_t launch_gemm_type(const GemmArgs& a, hipStream_t stream) {
  const int m_tiles = (a.M + kBM - 1) / kBM;
  // 128-wide weight tiles when they still give a workgroup per CU, else 64;
  // the grid is rounded up to a multiple of the 8 XCDs (extra workgroups exit)
  const bool wide = static_cast<int64_t>(m_tiles) * ((a.N + 127) / 128) >= 256;
  const int tiles = m_tiles * ((a.N + (wide ? 127 : 63)) / (wide ? 128 : 64));
  const uint32_t grid = static_cast<uint32_t>((tiles + 7) / 8 * 8);
  if (wide)
    gemm_kernel<TYPE, 128><<<grid, kGemmThreads, 0, stream>>>(a, tiles);
  else
    gemm_kernel<TYPE, 64><<<grid, kGemmThreads, 0, stream>>>(a, tiles);
  return hipGetLastError();
}

// Workspace: hi [M x K] and lo [M x K] fp16 planes, row scales [M] fp32, then
// (16-byte aligned) the sub-block sums, 32 bytes per (row, 256 values).
struct WorkspaceLayout {
  _Float16* hi;
  _Float16* lo;
  float* row_scale;
  _Float16* xs;
};

size_t xsum_offset(int64_t M, int64_t K) {
  const size_t bytes = static_cast<size_t>(M) * static_cast<size_t>(K) * 4 + static_cast<size_t>(M) * 4;
  return (bytes + 15) & ~size_t{15};
}

WorkspaceLayout layout(void* workspace, int64_t M, int64_t K) {
  auto* base = static_cast<_Float16*>(workspace);
  return {base, base + M * K, reinterpret_cast<float*>(base + 2 * M * K),
          reinterpret_cast<_Float16*>(static_cast<char*>(workspace) + xsum_offset(M, K))};
}

}  // namespace

size_t gemm_workspace_bytes(int64_t M, int64_t K) {
  const size_t bytes = xsum_offset(M, K) + static_cast<size_t>(M) * static_cast<size_t>(K / 256) * 32;
  return (bytes + 255) & ~size_t{255};
}

hipError_t launch_gemm_prep(const float* x, int64_t M, int64_t K, void* workspace,
                            hipStream_t stream) {
  const WorkspaceLayout ws = layout(workspace, M, K);
  prep_rows_kernel<<<static_cast<uint32_t>(M), 256, 0, stream>>>(x, ws.hi, ws.lo, ws.row_scale,
                                                                  ws.xs, static_cast<int>(K));
  return hipGetLastError();
}

hipError_t launch_gemm_core(const void* workspace, const void* w, int type, int64_t K, int64_t N,
                            float* y, int64_t M, hipStream_t stream) {
  const WorkspaceLayout ws = layout(const_cast<void*>(workspace), M, K);
  if (type == QK_TYPE_Q4_K && gemm_q4k_fits(M, K, N))
    return launch_gemm_q4k(ws.hi, ws.row_scale, ws.xs, w, K, N, y, M, stream);
  const GemmArgs a{ws.hi, ws.lo, ws.row_scale, static_cast<const uint8_t*>(w), y,
                   static_cast<int>(M), static_cast<int>(N), static_cast<int>(K)};
  return type == QK_TYPE_Q4_K ? launch_gemm_type<QK_TYPE_Q4_K>(a, stream)
                              : launch_gemm_type<QK_TYPE_Q6_K>(a, stream);
}

}  // namespace qk
