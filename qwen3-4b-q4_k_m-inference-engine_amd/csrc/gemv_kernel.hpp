// Streaming Q4_K / Q6_K mat-vec kernel templates (M <= 8 activation rows).
//
// Replaces quantize + project<Q4_K/Q6_K> (src/cuda/matmul.cu:8-22, 86-125),
// which run one 128-thread block per output element after a separate
// quantize launch. Here one persistent launch does both:
//   1. prologue: the workgroup quantises the fp32 activations into Q8 blocks
//      in LDS (or copies caller-provided Q8 blocks), while each wave's first
//      weight loads are already in flight;
//   2. each wave64 is an independent worker that streams whole row units:
//      lane = (row rr = lane / LPR, c = lane % LPR) with c -> (superblock
//      offset c/8, Q8 block c%8), so the LPR lanes of a row cover LPR/8
//      superblocks per iteration and every wave-wide load reads 64/LPR rows x
//      LPR/8 whole superblocks. Loads of U iterations are issued before the
//      first dot; lanes of a row reduce with DPP/shuffles; no barriers after
//      the prologue.
// Several weight segments sharing the input (attn q/k/v, src/Engine.cpp:83-85)
// run in one launch; the FFN mode computes gate and up for the same rows and
// writes SiLU(gate)*up (src/Engine.cpp:98-100, src/cuda/silu_multiply.cu:10).
#pragma once

#include <type_traits>

#include "qk_device.hpp"
#include "qk_launch.hpp"

namespace qk {

template <int TYPE>
struct WeightFrag;
template <>
struct WeightFrag<QK_TYPE_Q4_K> {
  using type = Q4KFrag;
  static constexpr int kBytes = kQ4KBytes;
  static __device__ __forceinline__ Q4KFrag load(const uint8_t* sb, uint32_t c) {
    return load_q4k(sb, c);
  }
  static __device__ __forceinline__ float dot(const Q4KFrag& w, const XFrag& x, uint32_t c) {
    return dot_q4k(w, x, c);
  }
};
template <>
struct WeightFrag<QK_TYPE_Q6_K> {
  using type = Q6KFrag;
  static constexpr int kBytes = kQ6KBytes;
  static __device__ __forceinline__ Q6KFrag load(const uint8_t* sb, uint32_t c) {
    return load_q6k(sb, c);
  }
  static __device__ __forceinline__ float dot(const Q6KFrag& w, const XFrag& x, uint32_t c) {
    return dot_q6k(w, x, c);
  }
};

// Q8 of one group of 8 consecutive activations per lane; the 4 lanes of a
// quad form one 32-activation block. code = roundf(RN(x/amax)*127) with the
// quotient from the correctly rounded reciprocal plus one Markstein
// correction step, which equals the IEEE quotient whenever the code can be
// non-zero (2^-64 <= amax <= 2^64); other amax take the IEEE division.
__device__ __forceinline__ void quantize_group(const float (&v)[8], qk_q8_block* blk, uint32_t q) {
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
  amax = fmaxf(amax, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                         0, __builtin_bit_cast(int, amax), 0xB1, 0xF, 0xF, false)));
  amax = fmaxf(amax, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                         0, __builtin_bit_cast(int, amax), 0x4E, 0xF, 0xF, false)));
  int code[8];
  if (amax == 0.0f) {
#pragma unroll
    for (int i = 0; i < 8; ++i) code[i] = 0;
  } else if (amax >= 0x1p-64f && amax <= 0x1p64f) {
    const float r = 1.0f / amax;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float q0 = v[i] * r;
      const float e = __builtin_fmaf(-q0, amax, v[i]);
      const float quotient = __builtin_fmaf(e, r, q0);
      code[i] = static_cast<int>(roundf(quotient * 127.0f));
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) code[i] = static_cast<int>(roundf((v[i] / amax) * 127.0f));
  }
  uint32_t lo = 0, hi = 0;
  int sum = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    lo |= (static_cast<uint32_t>(code[i]) & 0xFFu) << (8 * i);
    hi |= (static_cast<uint32_t>(code[i + 4]) & 0xFFu) << (8 * i);
    sum += code[i] + code[i + 4];
  }
  *reinterpret_cast<uint2*>(blk->codes + 8 * q) = make_uint2(lo, hi);
  // lanes 0,1 of the quad hold codes 0..15, lanes 2,3 codes 16..31
  const int pair = sum + __builtin_amdgcn_update_dpp(0, sum, 0xB1, 0xF, 0xF, false);
  const int other = __builtin_amdgcn_update_dpp(0, pair, 0x4E, 0xF, 0xF, false);
  if (q == 0) {
    const float scale = amax / 127.0f;
    blk->scale = scale;
    blk->scaled_sum = scale * static_cast<float>(pair + other);
    blk->neg32_sum_lo = -32 * pair;
    blk->neg32_sum_hi = -32 * other;
  }
}

// The prologue quantises fp32 x[M x K] into LDS Q8 blocks [MT][K/32] (rows
// m >= M are zero), 8 activations per task, tasks strided over the 256
// threads. The loads of a thread's first kStaged tasks are issued before the
// weight prefetch (global loads complete in issue order, so activations
// loaded after the prefetch would wait for all of it); further tasks load
// and quantise afterwards.
template <int MT>
struct XStage {
  static constexpr int kStaged = MT == 1 ? 5 : MT == 2 ? 3 : 2;
  f32x4 a[kStaged], b[kStaged];
};

// Loads of every staged task are unconditional (indices clamped into the
// buffer, rows m >= M selected to zero afterwards): a load under a branch
// would make the compiler's wait-count tracking assume nothing was issued
// after it and wait for the whole weight prefetch before the quantisation.
template <int MT>
__device__ __forceinline__ void load_x_group(const float* __restrict__ x, int M, int K, int t,
                                             f32x4& a, f32x4& b) {
  const int groups = K / 8;
  const int m = t / groups;
  const float* p = x + static_cast<int64_t>(min(m, M - 1)) * K + 8 * (t - m * groups);
  a = *reinterpret_cast<const f32x4_a4*>(p);
  b = *reinterpret_cast<const f32x4_a4*>(p + 4);
}

template <int MT>
__device__ __forceinline__ void stage_x(const float* __restrict__ x, int M, int K, XStage<MT>& st) {
  const int tasks = MT * (K / 8);
#pragma unroll
  for (int i = 0; i < XStage<MT>::kStaged; ++i) {
    const int t = min(static_cast<int>(threadIdx.x) + 256 * i, tasks - 1);
    load_x_group<MT>(x, M, K, t, st.a[i], st.b[i]);
  }
}

__device__ __forceinline__ void quantize_task(f32x4 a, f32x4 b, bool zero, int t,
                                              qk_q8_block* __restrict__ lds) {
  if (zero) {
    a = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    b = a;
  }
  const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  // task t covers activations 8t..8t+7 of the [MT][K] stream: block t/4, quarter t%4
  quantize_group(v, lds + t / 4, static_cast<uint32_t>(t & 3));
}

// K/8 is a multiple of 32, so the 4 lanes of a quad are always in or out together.
template <int MT>
__device__ void quantize_into_lds(const float* __restrict__ x, int M, int K, const XStage<MT>& st,
                                  qk_q8_block* __restrict__ lds) {
  const int groups = K / 8;
  const int tasks = MT * groups;
#pragma unroll
  for (int i = 0; i < XStage<MT>::kStaged; ++i) {
    const int t = static_cast<int>(threadIdx.x) + 256 * i;
    if (t < tasks) quantize_task(st.a[i], st.b[i], t / groups >= M, t, lds);
  }
  for (int t = static_cast<int>(threadIdx.x) + 256 * XStage<MT>::kStaged; t < tasks; t += 256) {
    f32x4 a, b;
    load_x_group<MT>(x, M, K, t, a, b);
    quantize_task(a, b, t / groups >= M, t, lds);
  }
}

// Caller-provided Q8 blocks [M][K/32] -> LDS [MT][K/32]; rows m >= M are zero.
template <int MT>
__device__ void copy_q8_into_lds(const qk_q8_block* __restrict__ q8, int M, int K,
                                 qk_q8_block* __restrict__ lds) {
  const int per_row = (K / 32) * 3;  // 16-byte chunks
  const u32x4* src = reinterpret_cast<const u32x4*>(q8);
  u32x4* dst = reinterpret_cast<u32x4*>(lds);
  for (int t = threadIdx.x; t < MT * per_row; t += blockDim.x) {
    const int m = t / per_row;
    dst[t] = m < M ? src[t] : u32x4{0u, 0u, 0u, 0u};
  }
}

template <int LPR>
__device__ __forceinline__ float row_lanes_sum(float v) {
  v = octet_sum(v);
  if constexpr (LPR >= 16) v += __shfl_xor(v, 8);
  if constexpr (LPR >= 32) v += __shfl_xor(v, 16);
  if constexpr (LPR >= 64) v += __shfl_xor(v, 32);
  return v;
}

// Loads of one chunk of a row: U iterations of LPR/8 superblocks.
template <int TYPE, int LPR, int U>
__device__ __forceinline__ void issue_chunk(const uint8_t* __restrict__ wrow, int S, int s0,
                                            uint32_t c, typename WeightFrag<TYPE>::type (&wf)[U]) {
  using WF = WeightFrag<TYPE>;
  constexpr int kSPI = LPR / 8;
  const int sbo = static_cast<int>(c >> 3);
#pragma unroll
  for (int i = 0; i < U; ++i) {
    const int s = min(s0 + i * kSPI + sbo, S - 1);
    wf[i] = WF::load(wrow + s * WF::kBytes, c & 7u);
  }
}

// acc[m] += the chunk's dots against activation row m.
template <int TYPE, int MT, int LPR, int U>
__device__ __forceinline__ void consume_chunk(const typename WeightFrag<TYPE>::type (&wf)[U],
                                              const qk_q8_block* __restrict__ xq, int S, int s0,
                                              uint32_t c, float (&acc)[MT]) {
  using WF = WeightFrag<TYPE>;
  constexpr int kSPI = LPR / 8;
  const uint32_t blk = c & 7u;
  const int sbo = static_cast<int>(c >> 3);
#pragma unroll
  for (int i = 0; i < U; ++i) {
    const int s = s0 + i * kSPI + sbo;
    const bool valid = s < S;
    const int sc = min(s, S - 1);
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      const XFrag xf = load_x(xq + m * S * 8 + sc * 8 + static_cast<int>(blk));
      const float v = WF::dot(wf[i], xf, blk);
      acc[m] += valid ? v : 0.0f;
    }
  }
}

// acc[m] += this lane's share of row `wrow` . x_m over all S superblocks; with
// `have_first` the first chunk's loads were issued by the caller into wf.
template <int TYPE, int MT, int LPR, int U>
__device__ __forceinline__ void stream_row(const uint8_t* __restrict__ wrow,
                                           const qk_q8_block* __restrict__ xq, int S, uint32_t c,
                                           float (&acc)[MT], typename WeightFrag<TYPE>::type (&wf)[U],
                                           bool have_first) {
  constexpr int kStep = (LPR / 8) * U;
  for (int s0 = 0; s0 < S; s0 += kStep) {
    if (!(have_first && s0 == 0)) issue_chunk<TYPE, LPR, U>(wrow, S, s0, c, wf);
    // keep every weight load of the chunk ahead of the first dot
    __builtin_amdgcn_sched_barrier(0);
    consume_chunk<TYPE, MT, LPR, U>(wf, xq, S, s0, c, acc);
  }
}

template <int MT, int LPR, int U>
__device__ __forceinline__ void stream_row_any(int type, const uint8_t* wrow,
                                               const qk_q8_block* xq, int S, uint32_t c,
                                               float (&acc)[MT]) {
  if (type == QK_TYPE_Q4_K) {
    Q4KFrag wf[U];
    stream_row<QK_TYPE_Q4_K, MT, LPR, U>(wrow, xq, S, c, acc, wf, false);
  } else {
    Q6KFrag wf[U];
    stream_row<QK_TYPE_Q6_K, MT, LPR, U>(wrow, xq, S, c, acc, wf, false);
  }
}

// MODE 0: y_j = x . W_j^T for every segment. MODE 1: segments 0/1 are gate
// and up of the same shape; h = SiLU(x . gate^T) * (x . up^T).
// TYPE: the weight type of every segment, or 0 when they differ (then the
// type is read per unit and the first chunk is not prefetched).
template <int MT, int LPR, int U, int MODE, int TYPE>
__global__ __launch_bounds__(256) void matvec_kernel(const MatvecParams p) {
  extern __shared__ __align__(16) unsigned char lds_raw[];
  qk_q8_block* xq = reinterpret_cast<qk_q8_block*>(lds_raw);
  constexpr int kRPU = 64 / LPR;  // rows per unit
  constexpr int kPre = TYPE == 0 ? QK_TYPE_Q4_K : TYPE;
  const int S = p.S;
  const uint32_t lane = threadIdx.x & 63u;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int rr = static_cast<int>(lane) / LPR;
  const uint32_t c = lane % LPR;
  const int nworkers = static_cast<int>(gridDim.x) * 4;
  const int first = static_cast<int>(blockIdx.x) * 4 + wave;

  auto unit_row = [&](int unit, int& j, int& row_raw, int& row) {
    j = 0;
#pragma unroll
    for (int t = 1; t < kMaxSegments; ++t)
      if (t < p.nseg && unit >= p.seg[t].unit_begin) j = t;
    row_raw = (unit - p.seg[j].unit_begin) * kRPU + rr;
    row = min(row_raw, p.seg[j].rows - 1);  // tail lanes re-read the last row
  };

  // Activation loads first, then the first chunk of this wave's first unit,
  // so the quantisation below runs while the weight loads are in flight.
  XStage<MT> stage;
  if (p.x) stage_x<MT>(p.x, p.M, p.K, stage);
  __builtin_amdgcn_sched_barrier(0);
  // Waves without a unit prefetch the last unit (in bounds, unused), so the
  // loads are issued on every path.
  typename WeightFrag<kPre>::type pre[U];
  const bool prefetched = TYPE != 0 && first < p.units;
  if constexpr (TYPE != 0) {
    int j, row_raw, row;
    unit_row(min(first, p.units - 1), j, row_raw, row);
    issue_chunk<TYPE, LPR, U>(p.seg[j].w + static_cast<int64_t>(row) * S * WeightFrag<TYPE>::kBytes,
                              S, 0, c, pre);
  }
  __builtin_amdgcn_sched_barrier(0);
  if (p.x)
    quantize_into_lds<MT>(p.x, p.M, p.K, stage, xq);
  else
    copy_q8_into_lds<MT>(p.q8, p.M, p.K, xq);
  __syncthreads();

  for (int unit = first; unit < p.units; unit += nworkers) {
    int j, row_raw, row;
    unit_row(unit, j, row_raw, row);
    const int rows = p.seg[j].rows;
    float acc[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[m] = 0.0f;
    if constexpr (TYPE == 0) {
      const int64_t row_bytes =
          static_cast<int64_t>(S) * (p.seg[j].type == QK_TYPE_Q4_K ? kQ4KBytes : kQ6KBytes);
      stream_row_any<MT, LPR, U>(p.seg[j].type, p.seg[j].w + row * row_bytes, xq, S, c, acc);
    } else {
      const int64_t row_bytes = static_cast<int64_t>(S) * WeightFrag<TYPE>::kBytes;
      stream_row<TYPE, MT, LPR, U>(p.seg[j].w + row * row_bytes, xq, S, c, acc, pre,
                                   prefetched && unit == first);
    }
    if constexpr (MODE == 0) {
#pragma unroll
      for (int m = 0; m < MT; ++m) acc[m] = row_lanes_sum<LPR>(acc[m]);
      if (c == 0 && row_raw < rows) {
#pragma unroll
        for (int m = 0; m < MT; ++m)
          if (m < p.M) p.seg[j].y[static_cast<int64_t>(m) * rows + row_raw] = acc[m];
      }
    } else {
      static_assert(MODE == 0 || TYPE != 0, "the FFN mode needs one weight type");
      float up[MT];
#pragma unroll
      for (int m = 0; m < MT; ++m) up[m] = 0.0f;
      const int64_t row_bytes = static_cast<int64_t>(S) * WeightFrag<kPre>::kBytes;
      stream_row<kPre, MT, LPR, U>(p.seg[1].w + row * row_bytes, xq, S, c, up, pre, false);
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        acc[m] = row_lanes_sum<LPR>(acc[m]);
        up[m] = row_lanes_sum<LPR>(up[m]);
      }
      if (c == 0 && row_raw < rows) {
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          const float g = acc[m];
          if (m < p.M) p.h[static_cast<int64_t>(m) * rows + row_raw] = (g / (1.0f + expf(-g))) * up[m];
        }
      }
    }
  }
}

using MatvecKernel = void (*)(MatvecParams);

// Kernel for MT activation rows, lanes per row `lpr`, unroll `u`, mode and
// weight type (0 = mixed); nullptr for a combination that is not built.
template <int MT>
MatvecKernel matvec_kernel_for(int lpr, int u, int mode, int type) {
  auto by_type = [&](auto lpr_c, auto u_c) -> MatvecKernel {
    constexpr int L = decltype(lpr_c)::value, UU = decltype(u_c)::value;
    if (mode == 1) {
      if (type == QK_TYPE_Q4_K) return &matvec_kernel<MT, L, UU, 1, QK_TYPE_Q4_K>;
      if (type == QK_TYPE_Q6_K) return &matvec_kernel<MT, L, UU, 1, QK_TYPE_Q6_K>;
      return nullptr;
    }
    if (type == QK_TYPE_Q4_K) return &matvec_kernel<MT, L, UU, 0, QK_TYPE_Q4_K>;
    if (type == QK_TYPE_Q6_K) return &matvec_kernel<MT, L, UU, 0, QK_TYPE_Q6_K>;
    return &matvec_kernel<MT, L, UU, 0, 0>;
  };
  using I8 = std::integral_constant<int, 8>;
  using I16 = std::integral_constant<int, 16>;
  using I32 = std::integral_constant<int, 32>;
  using I64 = std::integral_constant<int, 64>;
  using U2 = std::integral_constant<int, 2>;
  using U3 = std::integral_constant<int, 3>;
  using U5 = std::integral_constant<int, 5>;
  if (lpr == 8) return by_type(I8{}, U5{});
  if (lpr == 16) return by_type(I16{}, U5{});
  if (lpr == 32) return by_type(I32{}, U3{});
  if (u == 2) return by_type(I64{}, U2{});
  return by_type(I64{}, U5{});
}

}  // namespace qk
