// Streaming mat-vec kernels for up to 8 activation rows per launch.
#include "gemv_kernel.hpp"

namespace qk {

MatvecKernel matvec_kernel_m8(int lpr, int u, int mode, int type) {
  return matvec_kernel_for<8>(lpr, u, mode, type);
}

}  // namespace qk
