// Host launcher of the whole-share mat-vec (gemv_stream.hpp): one workgroup
// per CU, the CUs dealt to the segments in proportion to their bytes, each
// workgroup a contiguous range of rows. Used for M = 1 with fp32 activations
// whenever a workgroup's share of the weights fits in LDS; launch_matvec
// falls back to the streaming kernel otherwise.
#include <algorithm>
#include <map>
#include <mutex>
#include <utility>

#include "gemv_stream_mt.hpp"

namespace qk {

StreamMtKernel stream_mt_kernel_m4(int type, int J, int mode);
StreamMtKernel stream_mt_kernel_m8(int type, int J, int mode);

namespace {

template <int TYPE, int MODE>
StreamKernel stream_kernel_j(int J) {
  switch (J) {
    case 1: return &stream_matvec_kernel<TYPE, 1, MODE>;
    case 2: return &stream_matvec_kernel<TYPE, 2, MODE>;
    case 3: return &stream_matvec_kernel<TYPE, 3, MODE>;
    case 4: return &stream_matvec_kernel<TYPE, 4, MODE>;
    case 5: return &stream_matvec_kernel<TYPE, 5, MODE>;
    case 6: return &stream_matvec_kernel<TYPE, 6, MODE>;
    case 7: return &stream_matvec_kernel<TYPE, 7, MODE>;
    case 8: return &stream_matvec_kernel<TYPE, 8, MODE>;
    default: return nullptr;
  }
}

StreamKernel stream_kernel(int type, int J, int mode) {
  if (mode == 3) {
    if (type == QK_TYPE_Q4_K) return stream_kernel_j<QK_TYPE_Q4_K, 3>(J);
    if (type == QK_TYPE_Q6_K) return stream_kernel_j<QK_TYPE_Q6_K, 3>(J);
    return nullptr;
  }
  if (mode == 1) {
    if (type == QK_TYPE_Q4_K) return stream_kernel_j<QK_TYPE_Q4_K, 1>(J);
    if (type == QK_TYPE_Q6_K) return stream_kernel_j<QK_TYPE_Q6_K, 1>(J);
    return nullptr;
  }
  if (type == QK_TYPE_Q4_K) return stream_kernel_j<QK_TYPE_Q4_K, 0>(J);
  if (type == QK_TYPE_Q6_K) return stream_kernel_j<QK_TYPE_Q6_K, 0>(J);
  return stream_kernel_j<0, 0>(J);
}

std::mutex g_mutex;
std::map<int, std::pair<int, int>> g_device;        // device -> (CUs, LDS bytes per workgroup)
std::map<std::pair<const void*, int>, bool> g_lds;  // dynamic LDS limit set

}  // namespace

hipError_t device_limits(int& cus, int& max_lds) {
  int device = 0;
  hipError_t e = hipGetDevice(&device);
  if (e != hipSuccess) return e;
  std::lock_guard<std::mutex> lock(g_mutex);
  auto it = g_device.find(device);
  if (it == g_device.end()) {
    int c = 0, l = 0;
    e = hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, device);
    if (e != hipSuccess) return e;
    e = hipDeviceGetAttribute(&l, hipDeviceAttributeMaxSharedMemoryPerBlock, device);
    if (e != hipSuccess) return e;
    it = g_device.emplace(device, std::make_pair(c, l)).first;
  }
  cus = it->second.first;
  max_lds = it->second.second;
  return hipSuccess;
}

hipError_t allow_lds(const void* fn, int lds) {
  std::lock_guard<std::mutex> lock(g_mutex);
  const auto key = std::make_pair(fn, lds);
  if (g_lds.count(key)) return hipSuccess;
  const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  if (e == hipSuccess) g_lds.emplace(key, true);
  return e;
}

namespace {

int type_bytes(int type) { return type == QK_TYPE_Q4_K ? kQ4KBytes : kQ6KBytes; }

// Workgroups per segment in proportion to bytes, at least one, at most one
// per row, and no more than one per CU in all; false if segments outnumber CUs.
bool workgroup_counts(const MatvecParams& p, int nseg, int parts, int cus, int (&count)[kMaxSegments]) {
  double bytes[kMaxSegments] = {0.0}, total = 0.0;
  for (int j = 0; j < nseg; ++j) {
    bytes[j] = static_cast<double>(p.seg[j].rows) * p.S * type_bytes(p.seg[j].type) * parts;
    total += bytes[j];
  }
  if (nseg > cus) return false;
  int sum = 0;
  for (int j = 0; j < nseg; ++j) {
    const int want = static_cast<int>(cus * bytes[j] / total + 0.5);
    count[j] = std::clamp(want, 1, p.seg[j].rows);
    sum += count[j];
  }
  while (sum > cus) {  // trim the segment with the most workgroups
    int big = 0;
    for (int j = 1; j < nseg; ++j)
      if (count[j] > count[big]) big = j;
    --count[big];
    --sum;
  }
  return true;
}

// M = 2..8 (gemv_stream_mt.hpp): MT = 4 or 8 rows, every wave a run of whole
// rows; needs all MT * K / 8 activation tasks staged (4 per thread) and one
// weight type in all segments.
hipError_t launch_stream_mt(const MatvecParams& p, int mode, hipStream_t stream, bool& launched) {
  int cus = 0, max_lds = 0;
  hipError_t e = device_limits(cus, max_lds);
  if (e != hipSuccess) return e;
  const int MT = p.M <= 4 ? 4 : 8;
  if (MT * (p.K / 8) > 64 * kStreamWaves * kMtXStaged) return hipSuccess;
  const int nseg = mode == 1 ? 1 : p.nseg;
  const int parts = mode == 1 ? 2 : 1, wpp = kStreamWaves / parts;
  const int64_t S = p.S;
  for (int j = 1; j < nseg; ++j)
    if (p.seg[j].type != p.seg[0].type) return hipSuccess;  // one weight type per launch
  int count[kMaxSegments] = {0};
  if (!workgroup_counts(p, nseg, parts, cus, count)) return hipSuccess;

  StreamMtParams sp{};
  sp.x = p.x;
  sp.h = p.h;
  sp.M = p.M;
  sp.K = p.K;
  sp.S = p.S;
  sp.nseg = nseg;
  int64_t region = 16, sums = 0;
  int begin = 0;
  for (int j = 0; j < nseg; ++j) {
    const int per = p.seg[j].rows / count[j], rem = p.seg[j].rows % count[j];
    const int64_t rb = S * type_bytes(p.seg[j].type);
    const int64_t rows_max = per + (rem ? 1 : 0);
    const int64_t rpw = (rows_max + wpp - 1) / wpp;
    region = std::max<int64_t>(region, (2 + rpw * rb + 15) / 16 * 16);
    for (int64_t n : {static_cast<int64_t>(per), rows_max}) {  // the workgroups' row counts
      if (n == 0) continue;
      const int64_t groups = (n + 15) / 16;
      const int64_t ranges = std::min<int64_t>(S, std::max<int64_t>(1, (kStreamWaves + parts * groups - 1) / (parts * groups)));
      sums = std::max(sums, n * ranges * MT);
    }
    sp.seg[j] = {p.seg[j].w, p.seg[j].y, p.seg[j].rows, p.seg[j].type, begin, per, rem, 0};
    begin += count[j];
  }
  if (mode == 1) sp.seg[1] = {p.seg[1].w, nullptr, p.seg[1].rows, p.seg[1].type, 0, 0, 0, 0};
  const int64_t J = (region + 1023) / 1024;
  if (J > kStreamMaxJ) return hipSuccess;
  const int64_t lds = MT * S * 8 * static_cast<int64_t>(sizeof(qk_q8_block)) + kStreamWaves * region +
                      parts * sums * 4;
  if (lds > max_lds) return hipSuccess;
  sp.region = static_cast<int32_t>(region);
  sp.sums_stride = static_cast<int32_t>(sums);
  const int type = p.seg[0].type;
  const StreamMtKernel fn = MT == 4 ? stream_mt_kernel_m4(type, static_cast<int>(J), mode)
                                    : stream_mt_kernel_m8(type, static_cast<int>(J), mode);
  if (!fn) return hipSuccess;
  e = allow_lds(reinterpret_cast<const void*>(fn), static_cast<int>(lds));
  if (e != hipSuccess) return e;
  note("stream_mt_kernel", begin, MT, type, J, mode);
  hipLaunchKernelGGL(fn, dim3(static_cast<uint32_t>(begin)), dim3(64 * kStreamWaves),
                     static_cast<size_t>(lds), stream, sp);
  launched = true;
  return hipGetLastError();
}

}  // namespace

hipError_t launch_stream_matvec(const MatvecParams& p, int mode, hipStream_t stream, bool& launched) {
  launched = false;
  if (p.x == nullptr || (mode != 0 && mode != 1 && mode != 3) || p.M > 8) return hipSuccess;
  if (mode == 3 && (p.M != 1 || p.norm == nullptr)) return hipSuccess;  // the fold is M = 1 only
  if (p.M > 1) return launch_stream_mt(p, mode, stream, launched);
  if (p.K > kStreamMaxK) return hipSuccess;
  int cus = 0, max_lds = 0;
  hipError_t e = device_limits(cus, max_lds);
  if (e != hipSuccess) return e;
  const bool ffn = mode == 1 || mode == 3;
  const int nseg = ffn ? 1 : p.nseg;
  const int parts = ffn ? 2 : 1, wpp = kStreamWaves / parts;
  const int64_t S = p.S;

  int count[kMaxSegments] = {0};
  if (!workgroup_counts(p, nseg, parts, cus, count)) return hipSuccess;

  StreamParams sp{};
  sp.x = p.x;
  sp.h = p.h;
  sp.K = p.K;
  sp.S = p.S;
  sp.nseg = nseg;
  sp.norm = p.norm;
  sp.eps = p.eps;
  int J = 0, type = 0, begin = 0;
  int64_t max_sb = 0;
  bool q4 = false, q6 = false;
  for (int j = 0; j < nseg; ++j) {
    const int64_t rows_max = (p.seg[j].rows + count[j] - 1) / count[j];
    const int64_t sb = rows_max * S;
    const int64_t wave_bytes = 2 + (sb + wpp - 1) / wpp * type_bytes(p.seg[j].type);
    const int64_t chunks = (wave_bytes + 15) / 16;
    J = std::max<int>(J, static_cast<int>(std::min<int64_t>((chunks + 63) / 64, kStreamMaxJ + 1)));
    max_sb = std::max(max_sb, sb);
    (p.seg[j].type == QK_TYPE_Q4_K ? q4 : q6) = true;
    sp.seg[j] = {p.seg[j].w, p.seg[j].y, p.seg[j].rows, p.seg[j].type, begin,
                 p.seg[j].rows / count[j], p.seg[j].rows % count[j], 0};
    begin += count[j];
  }
  if (ffn) sp.seg[1] = {p.seg[1].w, nullptr, p.seg[1].rows, p.seg[1].type, 0, 0, 0, 0};
  if (J > kStreamMaxJ) return hipSuccess;
  type = q4 && q6 ? 0 : q4 ? QK_TYPE_Q4_K : QK_TYPE_Q6_K;
  sp.max_sb = static_cast<int32_t>(max_sb);
  // (mode 3: the wave partials of the row's sum of squares after the sums)
  const int64_t lds = S * 8 * static_cast<int64_t>(sizeof(qk_q8_block)) +
                      static_cast<int64_t>(kStreamWaves) * J * 1024 + parts * max_sb * 4 +
                      (mode == 3 ? 4 * kStreamWaves : 0);
  if (lds > max_lds) return hipSuccess;
  const StreamKernel fn = stream_kernel(type, J, mode);
  if (!fn) return hipSuccess;
  e = allow_lds(reinterpret_cast<const void*>(fn), static_cast<int>(lds));
  if (e != hipSuccess) return e;
  note("stream_matvec_kernel", begin, type, J, mode);
  hipLaunchKernelGGL(fn, dim3(static_cast<uint32_t>(begin)), dim3(64 * kStreamWaves),
                     static_cast<size_t>(lds), stream, sp);
  launched = true;
  return hipGetLastError();
}

}  // namespace qk
