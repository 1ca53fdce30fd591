// Streaming mat-vec kernels for up to 1 activation row per launch.
#include "gemv_kernel.hpp"

namespace qk {

MatvecKernel matvec_kernel_m1(int lpr, int u, int mode, int type) {
  return matvec_kernel_for<1>(lpr, u, mode, type);
}

}  // namespace qk
