// Fused FFN kernels (ffn_fused.hpp): Q4_K gate/up, Q4_K down, RMSNorm folded, for the
// share depths the launcher rounds to (16-byte chunks per lane of the
// gate/up share, JG, and of the down share, JD).
#include "ffn_fused.hpp"

namespace qk {

FfnKernel ffn_kernel_q4_norm(int jg, int jd, int pd) {
#define QK_FFN(JG, JD) \
  if (jg == JG && jd == JD && pd == 0) return &ffn_fused_kernel<QK_TYPE_Q4_K, JG, QK_TYPE_Q4_K, JD, 0, true>;
  QK_FFN(2, 2) QK_FFN(2, 4) QK_FFN(2, 6) QK_FFN(2, 8)
  QK_FFN(4, 2) QK_FFN(4, 4) QK_FFN(4, 6) QK_FFN(4, 8)
  QK_FFN(6, 2) QK_FFN(6, 4) QK_FFN(6, 6) QK_FFN(6, 8)
  QK_FFN(7, 2) QK_FFN(7, 4) QK_FFN(7, 6)
  QK_FFN(8, 2) QK_FFN(8, 4) QK_FFN(8, 6)
#undef QK_FFN
  return nullptr;
}

}  // namespace qk
