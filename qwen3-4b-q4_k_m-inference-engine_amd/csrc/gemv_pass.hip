// Host launcher of the multi-pass whole-share mat-vec (gemv_pass.hpp): M = 1,
// one weight matrix, fp32 activations, when a workgroup's share of the
// weights does not fit in LDS (MODE 0) and for every lm_head + argmax
// (MODE 2). One workgroup per CU.
#include <algorithm>

#include "gemv_pass.hpp"
#include "qk_launch.hpp"

namespace qk {
namespace {

template <int TYPE, int MODE>
PassKernel pass_kernel_j(int J) {
  switch (J) {
    case 4: return &pass_matvec_kernel<TYPE, MODE, 4>;
    case 5: return &pass_matvec_kernel<TYPE, MODE, 5>;
    case 6: return &pass_matvec_kernel<TYPE, MODE, 6>;
    case 7: return &pass_matvec_kernel<TYPE, MODE, 7>;
    case 8: return &pass_matvec_kernel<TYPE, MODE, 8>;
    default: return nullptr;
  }
}

PassKernel pass_kernel(int type, int mode, int J) {
  if (type == QK_TYPE_Q4_K) return mode == 2 ? pass_kernel_j<QK_TYPE_Q4_K, 2>(J) : pass_kernel_j<QK_TYPE_Q4_K, 0>(J);
  if (type == QK_TYPE_Q6_K) return mode == 2 ? pass_kernel_j<QK_TYPE_Q6_K, 2>(J) : pass_kernel_j<QK_TYPE_Q6_K, 0>(J);
  return nullptr;
}

}  // namespace

// Rows per pass and loads per lane: the pair that reads the fewest wasted
// chunk bytes per pass (ties: fewer loads), with R * row_bytes plus the 2
// alignment bytes within J KB, at most 16 rows (a quad per row) and
// kPassSums superblocks per pass. False if no row fits in kPassMaxJ KB.
bool pass_plan(int64_t S, int type, int& R, int& J) {
  const int64_t rb = S * (type == QK_TYPE_Q4_K ? kQ4KBytes : kQ6KBytes);
  double best = 0.0;
  R = J = 0;
  for (int j = 4; j <= kPassMaxJ; ++j) {
    const int64_t r = std::min<int64_t>({16, kPassSums / S, (1024 * j - 2) / rb});
    if (r < 1) continue;
    const double eff = static_cast<double>(r * rb) / (1024.0 * j);
    if (eff > best + 1e-9) {
      best = eff;
      R = static_cast<int>(r);
      J = j;
    }
  }
  return R > 0;
}

hipError_t launch_pass_matvec(const MatvecParams& p, int mode, hipStream_t stream, bool& launched) {
  launched = false;
  if (p.x == nullptr || p.M != 1 || p.nseg != 1 || (mode != 0 && mode != 2)) return hipSuccess;
  if (p.K > kStreamMaxK) return hipSuccess;
  const int type = p.seg[0].type;
  if (type != QK_TYPE_Q4_K && type != QK_TYPE_Q6_K) return hipSuccess;
  int R = 0, J = 0;
  if (!pass_plan(p.S, type, R, J)) return hipSuccess;
  int cus = 0, max_lds = 0;
  hipError_t e = device_limits(cus, max_lds);
  if (e != hipSuccess) return e;
  const int64_t lds = static_cast<int64_t>(p.S) * 8 * static_cast<int64_t>(sizeof(qk_q8_block)) +
                      static_cast<int64_t>(kPassWaves) * J * 1024 + kPassWaves * kPassSums * 4;
  if (lds + 8 * (kPassWaves + 1) > max_lds) return hipSuccess;
  const PassKernel fn = pass_kernel(type, mode, J);
  if (!fn) return hipSuccess;
  const int grid = std::min(cus, kArgmaxSlots);  // MODE 2: one partial per workgroup
  const int64_t W = static_cast<int64_t>(grid) * kPassWaves;
  const int64_t N = p.seg[0].rows;
  PassParams pp{};
  pp.x = p.x;
  pp.w = p.seg[0].w;
  pp.y = p.seg[0].y;
  pp.argmax_ws = p.argmax_ws;
  pp.argmax_result = p.argmax_result;
  pp.K = p.K;
  pp.S = p.S;
  pp.N = static_cast<int32_t>(N);
  pp.R = R;
  pp.full = static_cast<int32_t>(N / (W * R));
  pp.rest = static_cast<int32_t>(N - static_cast<int64_t>(pp.full) * W * R);
  pp.npass = pp.full + (pp.rest > 0 ? 1 : 0);
  e = allow_lds(reinterpret_cast<const void*>(fn), static_cast<int>(lds));
  if (e != hipSuccess) return e;
  note("pass_matvec_kernel", grid, type, mode, J, R);
  hipLaunchKernelGGL(fn, dim3(static_cast<uint32_t>(grid)), dim3(64 * kPassWaves), static_cast<size_t>(lds),
                     stream, pp);
  launched = true;
  return hipGetLastError();
}

}  // namespace qk
