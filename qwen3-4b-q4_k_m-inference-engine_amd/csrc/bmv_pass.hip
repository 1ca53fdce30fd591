// Host launcher of the multi-pass batched mat-vec (bmv_pass.hpp): M = 2..8,
// one weight matrix of either type, fp32 activations, matrices tall enough
// that every wave of the launch owns at least two 16-row groups (the
// lm_head). One workgroup per CU.
#include "bmv_pass.hpp"
#include "qk_launch.hpp"

namespace qk {
namespace {

template <int TYPE>
BmvPassKernel bmv_pass_kernel_j(int J) {
  switch (J) {
    case 4: return &bmv_pass_kernel<TYPE, 4>;
    case 5: return &bmv_pass_kernel<TYPE, 5>;
    case 6: return &bmv_pass_kernel<TYPE, 6>;
    case 7: return &bmv_pass_kernel<TYPE, 7>;
    case 8: return &bmv_pass_kernel<TYPE, 8>;
    default: return nullptr;
  }
}

}  // namespace

// Columns per pass C and chunks per lane J: the pair that loads the fewest
// bytes per useful byte (ties: fewer chunks). A run of C superblocks starts
// up to 3 bytes past its dword boundary and a Q6_K field read looks up to 4
// bytes past a superblock, so a run takes ceil((C * B + 11) / 16) chunks.
bool bmv_pass_plan(int64_t S, int type, int& C, int& cpr, int& J) {
  const int64_t B = type == QK_TYPE_Q4_K ? kQ4KBytes : kQ6KBytes;
  double best = 0.0;
  C = cpr = J = 0;
  for (int64_t c = 1; c <= S; ++c) {
    const int64_t chunks = (c * B + 11 + 15) / 16;
    const int64_t j = (16 * chunks + 63) / 64;
    if (j > kBpMaxJ) break;
    if (j < 4) continue;
    const double eff = static_cast<double>(c * B) / static_cast<double>(16 * 64 * j);
    if (eff > best + 1e-9) {
      best = eff;
      C = static_cast<int>(c);
      cpr = static_cast<int>(chunks);
      J = static_cast<int>(j);
    }
  }
  return C > 0;
}

hipError_t launch_bmv_pass(const MatvecParams& p, int mode, hipStream_t stream, bool& launched) {
  launched = false;
  if (mode != 0 || p.M < 2 || p.M > 8 || p.nseg != 1 || p.x == nullptr) return hipSuccess;
  const int type = p.seg[0].type;
  if (type != QK_TYPE_Q4_K && type != QK_TYPE_Q6_K) return hipSuccess;
  const int64_t B = type == QK_TYPE_Q4_K ? kQ4KBytes : kQ6KBytes;
  const int64_t N = p.seg[0].rows, S = p.S;
  if (N * S * B + 16 > INT32_MAX) return hipSuccess;  // 32-bit buffer offsets
  int cus = 0, max_lds = 0;
  hipError_t e = device_limits(cus, max_lds);
  if (e != hipSuccess) return e;
  if ((N + 15) / 16 < 2 * static_cast<int64_t>(cus) * kBpWaves) return hipSuccess;  // tall matrices only
  int C = 0, cpr = 0, J = 0;
  if (!bmv_pass_plan(S, type, C, cpr, J)) return hipSuccess;
  const int stride = static_cast<int>(p.K) + 16;
  const int act = bmv_ws_act_bytes(static_cast<int>(p.K));
  const int64_t lds = act + static_cast<int64_t>(kBpWaves) * J * 1024;
  if (lds > max_lds) return hipSuccess;
  const BmvPassKernel fn =
      type == QK_TYPE_Q4_K ? bmv_pass_kernel_j<QK_TYPE_Q4_K>(J) : bmv_pass_kernel_j<QK_TYPE_Q6_K>(J);
  if (!fn) return hipSuccess;
  BmvPassParams bp{};
  bp.x = p.x;
  bp.w = p.seg[0].w;
  bp.y = p.seg[0].y;
  bp.M = p.M;
  bp.K = static_cast<int32_t>(p.K);
  bp.S = static_cast<int32_t>(S);
  bp.N = static_cast<int32_t>(N);
  bp.stride = stride;
  bp.act = act;
  bp.C = C;
  bp.cpr = cpr;
  bp.ppg = static_cast<int32_t>((S + C - 1) / C);
  e = allow_lds(reinterpret_cast<const void*>(fn), static_cast<int>(lds));
  if (e != hipSuccess) return e;
  note("bmv_pass_kernel", cus, type, J, C);
  hipLaunchKernelGGL(fn, dim3(static_cast<uint32_t>(cus)), dim3(64 * kBpWaves), static_cast<size_t>(lds), stream,
                     bp);
  launched = true;
  return hipGetLastError();
}

}  // namespace qk
