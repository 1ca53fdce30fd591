// Whole-share mat-vec kernels for up to 8 activation rows (gemv_stream_mt.hpp).
#include "gemv_stream_mt.hpp"

namespace qk {

namespace {

template <int TYPE, int MODE>
StreamMtKernel pick_j(int J) {
  switch (J) {
    case 1: return &stream_mt_kernel<8, TYPE, 1, MODE>;
    case 2: return &stream_mt_kernel<8, TYPE, 2, MODE>;
    case 3: return &stream_mt_kernel<8, TYPE, 3, MODE>;
    case 4: return &stream_mt_kernel<8, TYPE, 4, MODE>;
    case 5: return &stream_mt_kernel<8, TYPE, 5, MODE>;
    case 6: return &stream_mt_kernel<8, TYPE, 6, MODE>;
    case 7: return &stream_mt_kernel<8, TYPE, 7, MODE>;
    case 8: return &stream_mt_kernel<8, TYPE, 8, MODE>;
    default: return nullptr;
  }
}

}  // namespace

StreamMtKernel stream_mt_kernel_m8(int type, int J, int mode) {
  if (mode == 1) {
    if (type == QK_TYPE_Q4_K) return pick_j<QK_TYPE_Q4_K, 1>(J);
    if (type == QK_TYPE_Q6_K) return pick_j<QK_TYPE_Q6_K, 1>(J);
    return nullptr;
  }
  if (type == QK_TYPE_Q4_K) return pick_j<QK_TYPE_Q4_K, 0>(J);
  if (type == QK_TYPE_Q6_K) return pick_j<QK_TYPE_Q6_K, 0>(J);
  return nullptr;
}

}  // namespace qk
