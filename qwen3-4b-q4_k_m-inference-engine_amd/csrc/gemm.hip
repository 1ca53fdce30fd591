// Activation prep of the prefill GEMM (M > 8 activation rows) and its
// workspace; the GEMM itself is gemm_kquant.hip.
//
// prep_rows_kernel: per activation row, the Q8 round trip of x
// (MatmulReference.hpp:11-29: round(x/amax*127) * (amax/127) per 32 values),
// scaled by a power of two 2^s that brings the row's largest |x| into
// [2^14, 2^15), then split into two fp16 planes hi + lo with hi = fp16(v),
// lo = fp16(v - hi): 22 significant bits of v; and, per 32 values, 2^-5 times
// their sum, also as hi + lo (the Q4_K min-term operand).
#include "gemm_prep.hpp"
#include "qk_launch.hpp"

namespace qk {
namespace {

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
  uint32_t h[4], l[4];
  float sum;
  q8_scaled_planes(v, bmax, up, h, l, sum);
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

// Workspace: hi [M x K] and lo [M x K] fp16 planes, row scales [M] fp32, then
// (16-byte aligned) the sub-block sums, 32 bytes per (row, 256 values), then
// (256-byte aligned) the GEMM's partial products when it splits K.
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

size_t partial_offset(int64_t M, int64_t K) {
  const size_t bytes = xsum_offset(M, K) + static_cast<size_t>(M) * static_cast<size_t>(K / 256) * 32;
  return (bytes + 255) & ~size_t{255};
}

WorkspaceLayout layout(void* workspace, int64_t M, int64_t K) {
  auto* base = static_cast<_Float16*>(workspace);
  return {base, base + M * K, reinterpret_cast<float*>(base + 2 * M * K),
          reinterpret_cast<_Float16*>(static_cast<char*>(workspace) + xsum_offset(M, K))};
}

}  // namespace

size_t gemm_workspace_bytes(int64_t M, int64_t K, int type, int64_t N) {
  const size_t bytes = partial_offset(M, K) + gemm_kq_partial_bytes(type, M, K, N);
  return (bytes + 255) & ~size_t{255};
}

hipError_t launch_gemm_prep(const float* x, int64_t M, int64_t K, void* workspace,
                            hipStream_t stream, bool skip) {
  if (skip) return hipSuccess;  // every GEMM of the call forms its planes itself
  const WorkspaceLayout ws = layout(workspace, M, K);
  prep_rows_kernel<<<static_cast<uint32_t>(M), 256, 0, stream>>>(x, ws.hi, ws.lo, ws.row_scale,
                                                                  ws.xs, static_cast<int>(K));
  return hipGetLastError();
}

hipError_t launch_gemm_core(const float* x, const void* workspace, const void* w, int type, int64_t K,
                            int64_t N, float* y, int64_t M, hipStream_t stream) {
  const WorkspaceLayout ws = layout(const_cast<void*>(workspace), M, K);
  if (!gemm_kq_fits(M, K, N)) return hipErrorInvalidValue;
  float* partials = reinterpret_cast<float*>(static_cast<char*>(const_cast<void*>(workspace)) +
                                             partial_offset(M, K));
  return launch_gemm_kq(type, x, ws.hi, ws.row_scale, ws.xs, w, K, N, y, M, partials, stream);
}

hipError_t launch_gemm_core_multi(const float* x, const void* workspace, const qk_segment* segments, int count,
                                  int64_t K, int64_t M, hipStream_t stream, bool& launched) {
  launched = false;
  const WorkspaceLayout ws = layout(const_cast<void*>(workspace), M, K);
  return launch_gemm_kq_multi(x, ws.hi, ws.row_scale, ws.xs, segments, count, K, M, stream, launched);
}

}  // namespace qk
