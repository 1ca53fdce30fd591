// Streaming mat-vec kernels for up to 1 activation row(s) per launch.
#include "gemv_kernel.hpp"

namespace qk {

MatvecKernel matvec_kernel_m1(int lpr, int mode, int type, bool q8in) {
  return matvec_kernel_for<1>(lpr, mode, type, q8in);
}

}  // namespace qk
