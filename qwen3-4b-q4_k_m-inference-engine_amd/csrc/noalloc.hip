// qk_matmul_noalloc: qk_matmul for callers that cannot allocate (code under
// graph capture, tight serving loops, harnesses that forbid hipMalloc). The
// prefill GEMM's workspace (activation planes, block sums, split-K partials)
// is a file-scope device array instead of a stream-ordered allocation.
//
// The array's name is a host-side stand-in, not a device address: the
// address is looked up once per device with hipGetSymbolAddress (the device
// current) and only that pointer reaches the kernels. Every call on one
// device shares that device's array, which keeps the last call's contents;
// nothing in it must start at zero (every byte a kernel reads is written by
// the same call first). Calls that overlap on one device race.
#include <hip/hip_runtime.h>

#include <mutex>

#include "qk_abi.h"
#include "qk_launch.hpp"

namespace qk {
namespace {

static __device__ __align__(256) unsigned char scratch[QK_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_mutex;
void* g_scratch[kMaxDevices] = {};

// The device address of this device's `scratch`, looked up on first use.
int scratch_pointer(void*& out) {
  int device = 0;
  hipError_t error = hipGetDevice(&device);
  if (error != hipSuccess) return set_error(QK_ERR_RUNTIME, "get device failed", error);
  if (device < 0 || device >= kMaxDevices)
    return set_error(QK_ERR_RUNTIME, "device index beyond the scratch table", hipSuccess);
  std::lock_guard<std::mutex> lock(g_mutex);
  if (!g_scratch[device]) {
    void* ptr = nullptr;
    error = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (error != hipSuccess || !ptr)
      return set_error(QK_ERR_RUNTIME, "scratch symbol lookup failed", error);
    g_scratch[device] = ptr;
  }
  out = g_scratch[device];
  return QK_OK;
}

}  // namespace
}  // namespace qk

extern "C" int qk_matmul_noalloc(const float* x, const void* w, int type, int64_t K, int64_t N,
                                 float* y, int64_t M, qk_stream_t stream) {
  // M <= 8 (and every shape qk_matmul rejects) needs no workspace: qk_matmul_ws
  // validates and runs it as qk_matmul does.
  const size_t need = qk_matmul_workspace_size(type, K, N, M);
  if (need == 0) return qk_matmul_ws(x, w, type, K, N, y, M, nullptr, 0, stream);
  if (need > QK_NOALLOC_SCRATCH_BYTES)
    return qk::set_error(QK_ERR_INVALID_ARGUMENT,
                         "matmul shape needs more workspace than the no-alloc scratch holds "
                         "(qk_matmul_workspace_size > QK_NOALLOC_SCRATCH_BYTES)",
                         hipSuccess);
  void* ptr = nullptr;
  const int status = qk::scratch_pointer(ptr);
  if (status != QK_OK) return status;
  return qk_matmul_ws(x, w, type, K, N, y, M, ptr, QK_NOALLOC_SCRATCH_BYTES, stream);
}
