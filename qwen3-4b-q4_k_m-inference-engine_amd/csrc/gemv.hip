// Q4_K / Q6_K mat-vec over raw GGUF superblocks and Q8 activation blocks.
//
// Replaces project<Q4_K/Q6_K> (src/cuda/matmul.cu:86-125), which runs one
// 128-thread block per output element. Here a wave64 owns 8 weight rows:
// lane = (row r = lane/8, block c = lane%8), so the 8 lanes of a row cover the
// 8 Q8 blocks (32 weights each) of a superblock and every wave-wide load
// reads 8 whole superblocks (Q4_K: one 128-byte line of qs per row). The
// KSPLIT waves of a workgroup split the superblocks of those 8 rows; each
// wave issues the loads of UNROLL superblocks before it consumes any, lanes
// reduce with DPP and waves through LDS. Activations enter as Q8 blocks read
// through L1/L2; the weight stream is the HBM traffic.
#include "qk_device.hpp"
#include "qk_launch.hpp"

namespace qk {
namespace {

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

// SB: superblocks per row (0 = runtime sb_rt). Each wave visits superblocks
// wave, wave+KSPLIT, ... in groups of UNROLL; out-of-range slots re-load the
// row's last superblock (in bounds) and contribute 0.
template <int TYPE, int SB, int KSPLIT, int UNROLL>
__global__ __launch_bounds__(64 * KSPLIT) void gemv_kernel(const uint8_t* __restrict__ w,
                                                           const qk_q8_block* __restrict__ q8,
                                                           float* __restrict__ y, int sb_rt,
                                                           int N) {
  using WF = WeightFrag<TYPE>;
  constexpr int kBytes = WF::kBytes;
  const int S = SB > 0 ? SB : sb_rt;
  const uint32_t lane = threadIdx.x & 63u;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const uint32_t r = lane >> 3;
  const uint32_t c = lane & 7u;
  const int row_raw = static_cast<int>(blockIdx.x) * 8 + static_cast<int>(r);
  const int row = row_raw < N ? row_raw : N - 1;  // tail rows re-read the last row
  const int64_t m = blockIdx.y;
  const uint8_t* wrow = w + static_cast<int64_t>(row) * S * kBytes;
  const qk_q8_block* xrow = q8 + m * S * 8 + c;

  float acc = 0.0f;
  const int slots = (S + KSPLIT - 1) / KSPLIT;  // superblocks per wave (rounded up)
  for (int i0 = 0; i0 < slots; i0 += UNROLL) {
    typename WF::type wf[UNROLL];
    XFrag xf[UNROLL];
#pragma unroll
    for (int i = 0; i < UNROLL; ++i) {
      int s = wave + (i0 + i) * KSPLIT;
      s = s < S ? s : S - 1;
      wf[i] = WF::load(wrow + s * kBytes, c);
      xf[i] = load_x(xrow + s * 8);
    }
    // keep every load of the group ahead of the first dot
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < UNROLL; ++i) {
      const float v = WF::dot(wf[i], xf[i], c);
      acc += (wave + (i0 + i) * KSPLIT < S) ? v : 0.0f;
    }
  }
  acc = octet_sum(acc);

  if constexpr (KSPLIT > 1) {
    __shared__ float partial[KSPLIT][8];
    if (c == 0) partial[wave][r] = acc;
    __syncthreads();
    if (wave != 0) return;
    acc = partial[0][r];
#pragma unroll
    for (int i = 1; i < KSPLIT; ++i) acc += partial[i][r];
  }
  if (c == 0 && row_raw < N) y[m * N + row_raw] = acc;
}

template <int TYPE, int SB, int KSPLIT, int UNROLL>
hipError_t launch_cfg(const qk_q8_block* q8, const uint8_t* w, int sb, int64_t N, float* y,
                      int64_t M, hipStream_t stream) {
  const dim3 grid(static_cast<uint32_t>((N + 7) / 8), static_cast<uint32_t>(M));
  gemv_kernel<TYPE, SB, KSPLIT, UNROLL><<<grid, dim3(64 * KSPLIT), 0, stream>>>(
      w, q8, y, sb, static_cast<int>(N));
  return hipGetLastError();
}

template <int TYPE>
hipError_t launch_type(const qk_q8_block* q8, const uint8_t* w, int64_t K, int64_t N, float* y,
                       int64_t M, hipStream_t stream) {
  const int sb = static_cast<int>(K / kQK);
  switch (sb) {  // Qwen3-4B widths 2560, 4096, 9728: every wave loads all its slots at once
    case 10: return launch_cfg<TYPE, 10, 5, 2>(q8, w, sb, N, y, M, stream);
    case 16: return launch_cfg<TYPE, 16, 8, 2>(q8, w, sb, N, y, M, stream);
    case 38: return launch_cfg<TYPE, 38, 8, 5>(q8, w, sb, N, y, M, stream);
    default: return launch_cfg<TYPE, 0, 4, 2>(q8, w, sb, N, y, M, stream);
  }
}

}  // namespace

hipError_t launch_gemv(const qk_q8_block* q8, const void* w, int type, int64_t K, int64_t N,
                       float* y, int64_t M, hipStream_t stream) {
  const auto* bytes = static_cast<const uint8_t*>(w);
  if (type == QK_TYPE_Q4_K) return launch_type<QK_TYPE_Q4_K>(q8, bytes, K, N, y, M, stream);
  return launch_type<QK_TYPE_Q6_K>(q8, bytes, K, N, y, M, stream);
}

}  // namespace qk
