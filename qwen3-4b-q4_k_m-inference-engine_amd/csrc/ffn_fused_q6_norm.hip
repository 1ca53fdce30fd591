// Fused FFN kernels (ffn_fused.hpp): Q4_K gate/up, Q6_K down, RMSNorm folded, for the
// share depths the launcher rounds to (16-byte chunks per lane of the
// gate/up share, JG, and of the down share, JD, and the Q6_K down
// pieces per lane unpacked ahead of h, PD).
#include "ffn_fused.hpp"

namespace qk {

FfnKernel ffn_kernel_q6_norm(int jg, int jd, int pd) {
#define QK_FFN(JG, JD, PD) \
  if (jg == JG && jd == JD && pd == PD) return &ffn_fused_kernel<QK_TYPE_Q4_K, JG, QK_TYPE_Q6_K, JD, PD, true>;
  QK_FFN(2, 2, 1) QK_FFN(2, 4, 1) QK_FFN(2, 4, 2) QK_FFN(2, 6, 2) QK_FFN(2, 8, 2) QK_FFN(2, 8, 3)
  QK_FFN(4, 2, 1) QK_FFN(4, 4, 1) QK_FFN(4, 4, 2) QK_FFN(4, 6, 2) QK_FFN(4, 8, 2) QK_FFN(4, 8, 3)
  QK_FFN(6, 2, 1) QK_FFN(6, 4, 1) QK_FFN(6, 4, 2) QK_FFN(6, 6, 2) QK_FFN(6, 8, 2) QK_FFN(6, 8, 3)
  QK_FFN(7, 2, 1) QK_FFN(7, 4, 1) QK_FFN(7, 4, 2) QK_FFN(7, 6, 2)
  QK_FFN(8, 2, 1) QK_FFN(8, 4, 1) QK_FFN(8, 4, 2) QK_FFN(8, 6, 2)
#undef QK_FFN
  return nullptr;
}

}  // namespace qk
