// Host launcher of the fused FFN block (ffn_fused.hpp): one workgroup per CU,
// h rows and y rows dealt evenly, share depths rounded up to an instantiated
// pair. Shapes that do not fit (share too deep for registers, LDS, more
// workgroups than rows, widths past the staging) are left to the caller's
// two-launch path.
#include <algorithm>

#include "ffn_fused.hpp"

namespace qk {

FfnKernel ffn_kernel_q4(int jg, int jd, int pd);
FfnKernel ffn_kernel_q4_norm(int jg, int jd, int pd);
FfnKernel ffn_kernel_q6(int jg, int jd, int pd);
FfnKernel ffn_kernel_q6_norm(int jg, int jd, int pd);

namespace {

// 200 ms of the 100 MHz real-time clock: far past any legitimate wait (the
// barrier completes within microseconds when every workgroup is resident).
constexpr uint32_t kSpinTicks = 20000000u;

int round_up_to(int j, std::initializer_list<int> choices) {
  for (int c : choices)
    if (j <= c) return c;
  return 0;
}

// 16-byte chunks per lane of a wave's share of at most `sb` superblocks of
// `bytes` each (2 bytes of dword alignment slack).
int share_depth(int64_t sb, int bytes) {
  const int64_t chunks = (2 + sb * bytes + 15) / 16;
  return static_cast<int>((chunks + 63) / 64);
}

}  // namespace

size_t ffn_sync_bytes() { return kFfnSyncBytes; }
size_t ffn_timeout_offset() { return kSyncTimeout * sizeof(uint32_t); }

hipError_t launch_ffn_fused(const FfnArgs& a, hipStream_t stream, bool& launched) {
  launched = false;
  if (a.gate_up_type != QK_TYPE_Q4_K) return hipSuccess;  // Q4_K gate/up only (the Q4_K_M layout)
  if (a.K > kStreamMaxK || a.N > kStreamMaxK || a.K % 256 || a.N % 256) return hipSuccess;
  int cus = 0, max_lds = 0;
  hipError_t e = device_limits(cus, max_lds);
  if (e != hipSuccess) return e;
  const int64_t G = cus;
  if (G > a.N || G > a.K) return hipSuccess;
  const int64_t S = a.K / 256, Sd = a.N / 256;
  const int BG = kQ4KBytes, BD = a.down_type == QK_TYPE_Q4_K ? kQ4KBytes : kQ6KBytes;
  const int64_t per = a.N / G, rem = a.N % G, dper = a.K / G, drem = a.K % G;
  const int64_t max_sb = (per + (rem ? 1 : 0)) * S, max_sbd = (dper + (drem ? 1 : 0)) * Sd;
  const int kWpp = kStreamWaves / 2, kDownWaves = kStreamWaves - kFfnHWaves;
  const int jg = round_up_to(share_depth((max_sb + kWpp - 1) / kWpp, BG), {2, 4, 6, 7, 8});
  const int64_t down_sb = (max_sbd + kDownWaves - 1) / kDownWaves;  // largest down share of a wave
  const int jd = round_up_to(share_depth(down_sb, BD), {2, 4, 6, 8});
  // Q6_K down: pieces per lane unpacked ahead of h (0: Q4_K, consumed after)
  const int pd = a.down_type == QK_TYPE_Q6_K ? round_up_to(static_cast<int>((4 * down_sb + 63) / 64), {1, 2, 3})
                                             : 0;
  if (jg == 0 || jd == 0 || (a.down_type == QK_TYPE_Q6_K && pd == 0) || jg + jd > 14) return hipSuccess;
  const int64_t q8 = static_cast<int64_t>(sizeof(qk_q8_block));
  const int64_t lds_a = S * 8 * q8 + kStreamWaves * jg * 1024 + 2 * max_sb * 4 + 4 * kStreamWaves;
  const int64_t lds_b = ffn_down_offset(static_cast<int>(S), jg, static_cast<int>(max_sb), static_cast<int>(Sd), jd) +
                        kStreamWaves * jd * 1024 + max_sbd * 4;
  const int64_t lds = std::max(lds_a, lds_b);
  if (lds > max_lds) return hipSuccess;
  const bool norm = a.norm != nullptr;
  FfnKernel fn = nullptr;
  if (a.down_type == QK_TYPE_Q4_K) fn = norm ? ffn_kernel_q4_norm(jg, jd, pd) : ffn_kernel_q4(jg, jd, pd);
  else if (a.down_type == QK_TYPE_Q6_K) fn = norm ? ffn_kernel_q6_norm(jg, jd, pd) : ffn_kernel_q6(jg, jd, pd);
  if (!fn) return hipSuccess;

  FfnParams p{};
  p.x = a.x;
  p.norm = a.norm;
  p.h = a.h;
  p.y = a.y;
  p.gate = static_cast<const uint8_t*>(a.gate);
  p.up = static_cast<const uint8_t*>(a.up);
  p.down = static_cast<const uint8_t*>(a.down);
  p.sync = static_cast<uint32_t*>(a.sync);
  p.K = static_cast<int32_t>(a.K);
  p.S = static_cast<int32_t>(S);
  p.N = static_cast<int32_t>(a.N);
  p.Sd = static_cast<int32_t>(Sd);
  p.per = static_cast<int32_t>(per);
  p.rem = static_cast<int32_t>(rem);
  p.dper = static_cast<int32_t>(dper);
  p.drem = static_cast<int32_t>(drem);
  p.max_sb = static_cast<int32_t>(max_sb);
  p.max_sbd = static_cast<int32_t>(max_sbd);
  p.eps = a.eps;
  p.spin_ticks = kSpinTicks;
  e = allow_lds(reinterpret_cast<const void*>(fn), static_cast<int>(lds));
  if (e != hipSuccess) return e;
  note("ffn_fused_kernel", G, QK_TYPE_Q4_K, jg, a.down_type, jd, pd, norm);
  hipLaunchKernelGGL(fn, dim3(static_cast<uint32_t>(G)), dim3(64 * kStreamWaves), static_cast<size_t>(lds),
                     stream, p);
  launched = true;
  return hipGetLastError();
}

}  // namespace qk
