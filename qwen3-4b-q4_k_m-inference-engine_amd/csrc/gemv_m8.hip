// Streaming mat-vec kernels for up to 8 activation row(s) per launch.
#include "gemv_kernel.hpp"

namespace qk {

MatvecKernel matvec_kernel_m8(int lpr, int mode, int type, bool q8in) {
  return matvec_kernel_for<8>(lpr, mode, type, q8in);
}

}  // namespace qk
