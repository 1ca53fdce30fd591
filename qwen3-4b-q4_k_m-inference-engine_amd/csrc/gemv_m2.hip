// Streaming mat-vec kernels for up to 2 activation rows per launch.
#include "gemv_kernel.hpp"

namespace qk {

MatvecKernel matvec_kernel_m2(int lpr, int u, int mode, int type) {
  return matvec_kernel_for<2>(lpr, u, mode, type);
}

}  // namespace qk
