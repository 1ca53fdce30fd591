// Whole-share batched mat-vec (bmv_ws.hpp): its instantiations and host
// launcher. M = 2..8 activation rows, one workgroup per CU, CUs dealt to the
// segments in proportion to their bytes, at most 16 rows per workgroup.
#include <algorithm>
#include <climits>

#include "bmv_ws.hpp"

namespace qk {

namespace {

int superblock_bytes(int type) { return type == QK_TYPE_Q4_K ? kQ4KBytes : kQ6KBytes; }

}  // namespace

BmvWsKernel bmv_ws_kernel_for(int type, int mode, bool q8in) {
  if (mode == 1) {
    if (q8in) return nullptr;
    if (type == QK_TYPE_Q4_K) return &bmv_ws_kernel<QK_TYPE_Q4_K, 1, false>;
    if (type == QK_TYPE_Q6_K) return &bmv_ws_kernel<QK_TYPE_Q6_K, 1, false>;
    return nullptr;
  }
  if (q8in) {
    if (type == QK_TYPE_Q4_K) return &bmv_ws_kernel<QK_TYPE_Q4_K, 0, true>;
    if (type == QK_TYPE_Q6_K) return &bmv_ws_kernel<QK_TYPE_Q6_K, 0, true>;
    return &bmv_ws_kernel<0, 0, true>;
  }
  if (type == QK_TYPE_Q4_K) return &bmv_ws_kernel<QK_TYPE_Q4_K, 0, false>;
  if (type == QK_TYPE_Q6_K) return &bmv_ws_kernel<QK_TYPE_Q6_K, 0, false>;
  return &bmv_ws_kernel<0, 0, false>;
}

// The plan of a launch (the CPU index model of the tests restates these
// rules). Returns false when the shape does not fit the kernel: more than 16
// rows per workgroup, a wave's run beyond kWsJ loads per lane, activations
// beyond the staged registers, or LDS.
bool bmv_ws_plan(const MatvecParams& p, int mode, int cus, int max_lds, BmvWsPlan& plan) {
  const int nseg = mode == 1 ? 1 : p.nseg;
  const int parts = mode == 1 ? 2 : 1;
  if (nseg < 1 || nseg > cus || p.M < 1 || p.M > 8) return false;
  double bytes[kMaxSegments] = {0.0}, total = 0.0;
  for (int j = 0; j < nseg; ++j) {
    bytes[j] = static_cast<double>(p.seg[j].rows) * p.S * superblock_bytes(p.seg[j].type) * parts;
    total += bytes[j];
  }
  int sum = 0;
  for (int j = 0; j < nseg; ++j) {
    plan.count[j] = std::clamp(static_cast<int>(cus * bytes[j] / total + 0.5), 1, p.seg[j].rows);
    sum += plan.count[j];
  }
  while (sum > cus) {  // trim the segment with the most workgroups
    int big = 0;
    for (int j = 1; j < nseg; ++j)
      if (plan.count[j] > plan.count[big]) big = j;
    --plan.count[big];
    --sum;
  }
  const int rpw = 16 / (kBmvWaves / parts);
  int rows_max = 0;
  plan.reg = 0;
  for (int j = 0; j < nseg; ++j) {
    rows_max = std::max(rows_max, (p.seg[j].rows + plan.count[j] - 1) / plan.count[j]);
    const int64_t row_bytes = static_cast<int64_t>(p.S) * superblock_bytes(p.seg[j].type);
    if ((2 + rpw * row_bytes + 15) / 16 > 64 * kWsJ) return false;
    plan.reg = std::max(plan.reg, bmv_ws_reg_bytes(rpw, static_cast<int>(row_bytes)));
  }
  if (rows_max > 16) return false;
  const int64_t staged = p.x != nullptr ? static_cast<int64_t>(p.M) * (p.K / 8) - 64 * kBmvWaves * kWsXStaged
                                        : static_cast<int64_t>(p.M) * (p.K / 32) - 64 * kBmvWaves * kWsQ8Staged;
  if (staged > 0) return false;
  plan.lds = bmv_ws_lds_bytes(p.K, parts, plan.reg);
  return plan.lds <= max_lds;
}

hipError_t launch_bmv_ws(const MatvecParams& p, int mode, hipStream_t stream, bool& launched) {
  launched = false;
  if (p.M < 2 || p.M > 8 || (mode != 0 && mode != 1)) return hipSuccess;
  const bool q8in = p.x == nullptr;
  if (q8in && (p.q8 == nullptr || mode != 0)) return hipSuccess;
  if (p.K > (INT32_MAX - 64) / 8) return hipSuccess;
  int cus = 0, max_lds = 0;
  hipError_t e = device_limits(cus, max_lds);
  if (e != hipSuccess) return e;
  BmvWsPlan plan{};
  if (!bmv_ws_plan(p, mode, cus, max_lds, plan)) return hipSuccess;

  const int nseg = mode == 1 ? 1 : p.nseg;
  BmvWsParams bp{};
  bp.x = p.x;
  bp.q8 = p.q8;
  bp.h = p.h;
  bp.M = p.M;
  bp.K = p.K;
  bp.S = p.S;
  bp.nseg = nseg;
  bp.stride = p.K + 16;
  bp.reg = plan.reg;
  bp.act = bmv_ws_act_bytes(p.K);
  bool q4 = false, q6 = false;
  int begin = 0;
  for (int j = 0; j < nseg; ++j) {
    bp.seg[j] = {p.seg[j].w, p.seg[j].y, p.seg[j].rows, p.seg[j].type, begin,
                 p.seg[j].rows / plan.count[j], p.seg[j].rows % plan.count[j], 0};
    (p.seg[j].type == QK_TYPE_Q4_K ? q4 : q6) = true;
    begin += plan.count[j];
  }
  if (mode == 1) bp.seg[1] = {p.seg[1].w, nullptr, p.seg[1].rows, p.seg[1].type, 0, 0, 0, 0};
  const int type = q4 && q6 ? 0 : q4 ? QK_TYPE_Q4_K : QK_TYPE_Q6_K;
  const BmvWsKernel fn = bmv_ws_kernel_for(type, mode, q8in);
  if (!fn) return hipSuccess;
  e = allow_lds(reinterpret_cast<const void*>(fn), plan.lds);
  if (e != hipSuccess) return e;
  note("bmv_ws_kernel", begin, type, mode, q8in, plan.reg);
  hipLaunchKernelGGL(fn, dim3(static_cast<uint32_t>(begin)), dim3(64 * kBmvWaves),
                     static_cast<size_t>(plan.lds), stream, bp);
  launched = true;
  return hipGetLastError();
}

}  // namespace qk
