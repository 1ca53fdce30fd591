// Host launcher of the streaming mat-vec (kernels in gemv_kernel.hpp,
// instantiated per activation-row count in gemv_m{1,2,4,8}.hip): orders the
// segments by type, sizes the grid (one workgroup per CU, split between the
// types of a mixed launch) and picks the lanes per row for the shape.
#include <algorithm>
#include <climits>
#include <cstdint>
#include <map>
#include <mutex>
#include <utility>

#include "gemv_kernel.hpp"

namespace qk {

MatvecKernel matvec_kernel_m1(int lpr, int mode, int type, bool q8in);
MatvecKernel matvec_kernel_m2(int lpr, int mode, int type, bool q8in);
MatvecKernel matvec_kernel_m4(int lpr, int mode, int type, bool q8in);
MatvecKernel matvec_kernel_m8(int lpr, int mode, int type, bool q8in);

namespace {

struct DeviceFacts {
  int cus = 0;
  size_t max_lds = 0;
};

std::mutex g_mutex;
std::map<int, DeviceFacts> g_devices;
std::map<std::pair<MatvecKernel, size_t>, int> g_occupancy;

hipError_t device_facts(DeviceFacts& out) {
  int device = 0;
  hipError_t e = hipGetDevice(&device);
  if (e != hipSuccess) return e;
  std::lock_guard<std::mutex> lock(g_mutex);
  auto it = g_devices.find(device);
  if (it == g_devices.end()) {
    DeviceFacts f;
    e = hipDeviceGetAttribute(&f.cus, hipDeviceAttributeMultiprocessorCount, device);
    if (e != hipSuccess) return e;
    int lds = 0;
    e = hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerBlock, device);
    if (e != hipSuccess) return e;
    f.max_lds = static_cast<size_t>(lds);
    it = g_devices.emplace(device, f).first;
  }
  out = it->second;
  return hipSuccess;
}

hipError_t blocks_per_cu(MatvecKernel fn, int threads, size_t lds, int& out) {
  std::lock_guard<std::mutex> lock(g_mutex);
  const auto key = std::make_pair(fn, lds);
  auto it = g_occupancy.find(key);
  if (it == g_occupancy.end()) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                       static_cast<int>(lds));
    if (e != hipSuccess) return e;
    int n = 0;
    e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, fn, threads, lds);
    if (e != hipSuccess) return e;
    it = g_occupancy.emplace(key, std::max(n, 1)).first;
  }
  out = it->second;
  return hipSuccess;
}

// Iterations on the busiest wave when groups of 64/lpr rows are dealt
// round-robin to `waves` waves, each row taking ceil(S / (lpr/4))
// iterations (twice that for gate + up).
int64_t wave_iterations(int64_t rows, int64_t waves, int lpr, int S, int mode) {
  const int64_t rpg = 64 / lpr, spi = lpr / 4;
  const int64_t groups = (rows + rpg - 1) / rpg;
  const int64_t ipu = (S + spi - 1) / spi * (mode == 1 ? 2 : 1);
  return (groups + waves - 1) / waves * ipu;
}

MatvecKernel pick_kernel(int mt, int lpr, int mode, int type, bool q8in) {
  switch (mt) {
    case 1: return matvec_kernel_m1(lpr, mode, type, q8in);
    case 2: return matvec_kernel_m2(lpr, mode, type, q8in);
    case 4: return matvec_kernel_m4(lpr, mode, type, q8in);
    default: return matvec_kernel_m8(lpr, mode, type, q8in);
  }
}

}  // namespace

int matvec_rows_per_launch(int64_t K) {
  DeviceFacts dev;
  if (device_facts(dev) != hipSuccess) return 0;
  const size_t per_row = static_cast<size_t>(K / 32) * sizeof(qk_q8_block);
  for (int rows : {8, 4, 2, 1})
    if (per_row * rows <= dev.max_lds) return rows;
  return 0;
}

hipError_t launch_matvec(MatvecParams p, int mode, hipStream_t stream) {
  // M = 2..8: the whole-share batched mat-vec on the matrix cores
  // (bmv_ws.hip), else (gate/up) the batched mat-vec (bmv.hip).
  bool launched = false;
  hipError_t e = launch_bmv_ws(p, mode, stream, launched);
  if (e != hipSuccess || launched) return e;
  e = launch_bmv(p, mode, stream, launched);
  if (e != hipSuccess || launched) return e;
  // very tall matrices (the lm_head) at M = 2..8: the multi-pass batched form
  e = launch_bmv_pass(p, mode, stream, launched);
  if (e != hipSuccess || launched) return e;
  // Shapes whose per-CU share fits in LDS take the whole-share kernel
  // (gemv_stream.hip).
  e = launch_stream_matvec(p, mode, stream, launched);
  if (e != hipSuccess || launched) return e;
  // Larger M = 1 shapes and the lm_head + argmax: the multi-pass form (gemv_pass.hip).
  e = launch_pass_matvec(p, mode, stream, launched);
  if (e != hipSuccess || launched) return e;
  DeviceFacts dev;
  e = device_facts(dev);
  if (e != hipSuccess) return e;
  const int M = p.M;
  const int mt = M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : 8;
  const int waves = mt == 1 ? matvec_waves<1>() : matvec_waves<8>();
  const size_t lds = static_cast<size_t>(mt) * static_cast<size_t>(p.K / 32) * sizeof(qk_q8_block);
  if (lds > dev.max_lds) return hipErrorInvalidValue;

  // Row space: the segments' rows back to back, Q4_K segments first (the
  // mixed kernel gives each type its own workgroups). The FFN mode streams
  // the gate rows; up is read alongside through seg[1].
  if (mode == 1) p.nseg = 1;
  std::stable_sort(p.seg, p.seg + p.nseg, [](const MatvecSegment& l, const MatvecSegment& r) {
    return l.type == QK_TYPE_Q4_K && r.type != QK_TYPE_Q4_K;
  });
  int64_t rows4 = 0, rows6 = 0, begin = 0;
  for (int j = 0; j < p.nseg; ++j) {
    p.seg[j].row_begin = static_cast<int32_t>(begin);
    begin += p.seg[j].rows;
    (p.seg[j].type == QK_TYPE_Q4_K ? rows4 : rows6) += p.seg[j].rows;
  }
  if (begin > INT32_MAX - 64) return hipErrorInvalidValue;
  p.rows_total = static_cast<int32_t>(begin);
  const int type = rows6 == 0 ? QK_TYPE_Q4_K : rows4 == 0 ? QK_TYPE_Q6_K : 0;

  // Workgroups: one per CU (times the occupancy), never more than rows; a
  // mixed launch splits them in proportion to each type's bytes.
  const MatvecKernel probe = pick_kernel(mt, 8, mode, type, p.x == nullptr);
  if (!probe) return hipErrorInvalidValue;
  int per_cu = 1;
  e = blocks_per_cu(probe, 64 * waves, lds, per_cu);
  if (e != hipSuccess) return e;
  int64_t grid = std::min<int64_t>(static_cast<int64_t>(dev.cus) * per_cu, begin);
  if (mode == 2) grid = std::min<int64_t>(grid, kArgmaxSlots);  // one partial per workgroup
  int64_t wg4 = grid;
  if (type == 0) {
    if (grid < 2) return hipErrorInvalidValue;  // rows_total >= 2 here
    const double b4 = static_cast<double>(rows4) * kQ4KBytes, b6 = static_cast<double>(rows6) * kQ6KBytes;
    wg4 = std::clamp<int64_t>(static_cast<int64_t>(grid * b4 / (b4 + b6) + 0.5), 1, grid - 1);
  }
  p.split_wg = static_cast<int32_t>(wg4);
  p.split_row = static_cast<int32_t>(rows4);

  // Lanes per row: the fewest iterations (weighted by superblock bytes) on
  // the busiest wave; ties go to the narrower row, whose reductions are shorter.
  int lpr = 64;
  int64_t best = INT64_MAX;
  for (int cand : {8, 16, 32, 64}) {
    int64_t cost = 0;
    if (rows4) cost = std::max(cost, wave_iterations(rows4, wg4 * waves, cand, p.S, mode) * kQ4KBytes);
    if (rows6)
      cost = std::max(cost, wave_iterations(rows6, (type == 0 ? grid - wg4 : grid) * waves, cand,
                                            p.S, mode) * kQ6KBytes);
    if (cost < best) {
      best = cost;
      lpr = cand;
    }
  }
  const MatvecKernel fn = pick_kernel(mt, lpr, mode, type, p.x == nullptr);
  if (!fn) return hipErrorInvalidValue;
  e = blocks_per_cu(fn, 64 * waves, lds, per_cu);  // sets the kernel's dynamic LDS limit
  if (e != hipSuccess) return e;
  note("matvec_kernel", grid, mt, lpr, mode, type, p.x == nullptr);
  hipLaunchKernelGGL(fn, dim3(static_cast<uint32_t>(grid)), dim3(64 * waves), lds, stream, p);
  return hipGetLastError();
}

}  // namespace qk
