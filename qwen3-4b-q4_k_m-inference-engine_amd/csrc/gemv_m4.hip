// Streaming mat-vec kernels for up to 4 activation rows per launch.
#include "gemv_kernel.hpp"

namespace qk {

MatvecKernel matvec_kernel_m4(int lpr, int u, int mode, int type) {
  return matvec_kernel_for<4>(lpr, u, mode, type);
}

}  // namespace qk
