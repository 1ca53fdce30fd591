// Host launcher of the streaming mat-vec (kernels in gemv_kernel.hpp,
// instantiated per activation-row count in gemv_m{1,2,4,8}.hip): picks the
// row unit and unroll for the shape, sizes a persistent grid from the
// kernel's occupancy so every wave gets the same number of row units.
#include <algorithm>
#include <map>
#include <mutex>
#include <utility>

#include "gemv_kernel.hpp"

namespace qk {

MatvecKernel matvec_kernel_m1(int lpr, int u, int mode, int type);
MatvecKernel matvec_kernel_m2(int lpr, int u, int mode, int type);
MatvecKernel matvec_kernel_m4(int lpr, int u, int mode, int type);
MatvecKernel matvec_kernel_m8(int lpr, int u, int mode, int type);

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

hipError_t blocks_per_cu(MatvecKernel fn, size_t lds, int& out) {
  std::lock_guard<std::mutex> lock(g_mutex);
  const auto key = std::make_pair(fn, lds);
  auto it = g_occupancy.find(key);
  if (it == g_occupancy.end()) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                       static_cast<int>(lds));
    if (e != hipSuccess) return e;
    int n = 0;
    e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, fn, 256, lds);
    if (e != hipSuccess) return e;
    it = g_occupancy.emplace(key, std::max(n, 1)).first;
  }
  out = it->second;
  return hipSuccess;
}

// Lanes per row: the narrowest row unit that still gives at least 8 units per
// compute unit (so every CU streams from several waves), then for 64 lanes the
// unroll depth that wastes fewer superblock slots.
void choose_shape(int S, int64_t rows_total, int cus, int& lpr, int& u) {
  lpr = 64;
  for (int cand : {8, 16, 32, 64}) {
    if (rows_total / (64 / cand) >= 8 * static_cast<int64_t>(cus)) {
      lpr = cand;
      break;
    }
  }
  u = lpr == 32 ? 3 : 5;
  if (lpr == 64) {
    auto waste = [&](int uu) { return (S + 8 * uu - 1) / (8 * uu) * (8 * uu) - S; };
    u = waste(5) <= waste(2) ? 5 : 2;
  }
}

MatvecKernel pick_kernel(int mt, int lpr, int u, int mode, int type) {
  switch (mt) {
    case 1: return matvec_kernel_m1(lpr, u, mode, type);
    case 2: return matvec_kernel_m2(lpr, u, mode, type);
    case 4: return matvec_kernel_m4(lpr, u, mode, type);
    default: return matvec_kernel_m8(lpr, u, mode, type);
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
  DeviceFacts dev;
  hipError_t e = device_facts(dev);
  if (e != hipSuccess) return e;
  const int M = p.M;
  const int mt = M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : 8;
  const size_t lds = static_cast<size_t>(mt) * static_cast<size_t>(p.K / 32) * sizeof(qk_q8_block);
  if (lds > dev.max_lds) return hipErrorInvalidValue;
  int64_t rows_total = 0;
  for (int j = 0; j < (mode == 0 ? p.nseg : 1); ++j) rows_total += p.seg[j].rows;
  int lpr = 8, u = 5;
  choose_shape(p.S, rows_total, dev.cus, lpr, u);
  int type = p.seg[0].type;
  for (int j = 1; j < p.nseg; ++j)
    if (p.seg[j].type != type) type = 0;
  const int rpu = 64 / lpr;
  int units = 0;
  for (int j = 0; j < p.nseg; ++j) {
    p.seg[j].unit_begin = units;
    if (mode == 0 || j == 0) units += (p.seg[j].rows + rpu - 1) / rpu;
    else p.seg[j].unit_begin = 0;
  }
  if (mode == 1) p.nseg = 1;  // units index gate rows; up is read alongside
  p.units = units;
  const MatvecKernel fn = pick_kernel(mt, lpr, u, mode, type);
  if (!fn) return hipErrorInvalidValue;
  int per_cu = 1;
  e = blocks_per_cu(fn, lds, per_cu);
  if (e != hipSuccess) return e;
  // as many waves as fit, but every wave gets the same number of units
  const int64_t max_workers = static_cast<int64_t>(dev.cus) * per_cu * 4;
  const int64_t per_worker = (units + max_workers - 1) / max_workers;
  const int64_t workers = (units + per_worker - 1) / per_worker;
  const uint32_t grid = static_cast<uint32_t>((workers + 3) / 4);
  hipLaunchKernelGGL(fn, dim3(grid), dim3(256), lds, stream, p);
  return hipGetLastError();
}

}  // namespace qk
