// Batched mat-vec kernel entry (bmv.hpp) and its host launcher: M = 2..8
// activation rows in fp32, one workgroup per CU, CUs dealt to the segments
// in proportion to their bytes.
#include <algorithm>
#include <climits>

#include "bmv.hpp"

namespace qk {

namespace {

// Workgroup owning row r of a segment cut as in bmv_kernel (per rows each,
// the first rem workgroups one more).
__device__ __forceinline__ int bmv_owner(int r, int per, int rem) {
  const int big = rem * (per + 1);
  return r < big ? r / (per + 1) : rem + (r - big) / per;
}

// Q8 of h (qk_ffn at M = 2..8) in the gate/up launch. Block b of h (values
// 32b..32b+31 of every activation row) spans the workgroups that own those
// rows. Each of them, once its h stores are performed at the memory side
// (agent-scope stores, then s_waitcnt vmcnt(0) and the workgroup barrier),
// adds 1 to the block's arrival counter (agent-scope atomic, performed at
// the memory side); the one whose add completes the owner count resets the
// counter for the next launch and quantises the block for every activation
// row, a quad per row, with the quantiser of quantize_q8_kernel (same codes
// and record bits). Its h loads are agent-scope loads issued after the
// atomic returned, so they read every owner's stores. No workgroup waits
// for another, so nothing assumes co-residency.
__device__ __forceinline__ void bmv_close_blocks(const BmvParams& p, const BmvShare& sh, int N,
                                                 unsigned char* lds_raw) {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's h stores are performed
  __syncthreads();                                   // ... and every thread's
  lds_u32* closes = (lds_u32*)(lds_raw);             // the activation codes are no longer read
  const int tid = static_cast<int>(threadIdx.x);
  const int b0 = sh.r0 >> 5, nb = ((sh.r0 + sh.nrows - 1) >> 5) - b0 + 1;
  const int per = sh.per, rem = sh.rem;
  if (tid < nb) {
    const int b = b0 + tid;
    const int owners = bmv_owner(min(32 * b + 31, N - 1), per, rem) - bmv_owner(32 * b, per, rem) + 1;
    const uint32_t seen =
        __hip_atomic_fetch_add(p.arrive + b, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
    const bool last = seen == static_cast<uint32_t>(owners);
    if (last) __hip_atomic_store(p.arrive + b, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    closes[tid] = last ? 1u : 0u;
  }
  __syncthreads();
  const int M = p.M, q = tid >> 2;  // quad q: block b0 + q / M, activation row q % M
  if (q >= nb * M) return;           // whole quads
  const int i = q / M, m = q - i * M;
  if (closes[i] == 0u) return;
  const int b = b0 + i;
  const float* src = p.h + static_cast<int64_t>(m) * N + 32 * b + 8 * (tid & 3);
  float v[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) v[k] = __hip_atomic_load(src + k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  store_q8_quarter(p.hq + static_cast<int64_t>(m) * (N / 32) + b, static_cast<uint32_t>(tid & 3),
                   quantize_quarter(v));
}

// One type's path of a workgroup: prefetch, quantise, stream, totals.
template <int TYPE, int MODE, int P>
__device__ __forceinline__ void bmv_body(const BmvParams& p, const BmvShare& sh, int rows_seg,
                                         float* yout, int groups_max, unsigned char* lds_raw) {
  constexpr int B = TYPE == QK_TYPE_Q4_K ? kQ4KBytes : kQ6KBytes;
  constexpr int kParts = MODE == 1 ? 2 : 1;
  constexpr int kBmvXStaged = TYPE == QK_TYPE_Q4_K ? kBmvXStaged4 : kBmvXStaged6;
  const int K = p.K, M = p.M, stride = p.stride;
  const int tid = static_cast<int>(threadIdx.x);
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  // activation tasks (8 values each): the first kBmvXStaged per lane load
  // ahead of the weights
  const int groups8 = K / 8, tasks = M * groups8;
  f32x4 xa[kBmvXStaged], xb[kBmvXStaged];
#pragma unroll
  for (int i = 0; i < kBmvXStaged; ++i)
    load_x_group(p.x, M, K, min(tid + 64 * kBmvWaves * i, tasks - 1), xa[i], xb[i]);
  __builtin_amdgcn_sched_barrier(0);

  // this wave's units [u_lo, u_hi) and its tile count
  const int units = kParts * sh.groups * sh.ranges;
  const int u_lo = units * wave / kBmvWaves, u_hi = units * (wave + 1) / kBmvWaves;
  int ntiles = 0;
  for (int u = u_lo; u < u_hi; ++u) {
    const int rr = u % sh.ranges;
    ntiles += sh.run_begin(rr + 1) - sh.run_begin(rr);
  }
  BmvCursor start;
  cursor_seek(start, sh, u_lo < u_hi ? u_lo : 0);
  start.left = ntiles;

  BmvLane L;
  L.n = lane & 15;
  L.kq = lane >> 4;
  L.zero = static_cast<uint32_t>(8 * stride);
  L.a4_valid = (L.n < 8) == (L.kq < 2);
  L.a4_base = static_cast<uint32_t>((L.n & 7) * stride + 16 * (L.kq & 1));
  L.a6_valid = (L.n >> 2) == L.kq;
  L.a6_base = static_cast<uint32_t>((L.n & 3) * stride + 16 * L.kq);

  // the first P tiles
  BmvTile<TYPE> buf[P];
  BmvCursor lc = start;
#pragma unroll
  for (int j = 0; j < P; ++j) {
    bmv_load(buf[j], bmv_sb<B>(sh, lc, L.n), L.kq);
    cursor_next(lc, sh);
  }
  __builtin_amdgcn_sched_barrier(0);

  lds_u8* codes = (lds_u8*)(lds_raw);
  lds_f32* xs = (lds_f32*)(lds_raw + bmv_lds_z(stride));
  lds_f32* xss = xs + K / 4;
  lds_f32* xf = xs + K / 2;
  lds_f32* sums = xs + K;
  // Chunk c = tasks tid + 64*kBmvWaves*(kBmvXStaged*c + i), i < kBmvXStaged;
  // chunk 0 is staged. Wider rows (8 x 4096, 8 x 9728) run the later chunks
  // two buffers deep: chunk c+1 loads while chunk c is quantised. The loads
  // are unconditional (clamped into x; a chunk past the end re-reads the last
  // task) so the waits count them exactly.
  constexpr int kChunk = 64 * kBmvWaves * kBmvXStaged;
  auto quantize_chunk = [&](const f32x4 (&a)[kBmvXStaged], const f32x4 (&b)[kBmvXStaged], int c) {
#pragma unroll
    for (int i = 0; i < kBmvXStaged; ++i) {
      const int t = tid + kChunk * c + 64 * kBmvWaves * i;
      if (t < tasks) bmv_quantize_task(a[i], b[i], t, groups8, stride, codes, xs, xss, xf);
    }
  };
  auto load_chunk = [&](f32x4 (&a)[kBmvXStaged], f32x4 (&b)[kBmvXStaged], int c) {
#pragma unroll
    for (int i = 0; i < kBmvXStaged; ++i)
      load_x_group(p.x, M, K, min(tid + kChunk * c + 64 * kBmvWaves * i, tasks - 1), a[i], b[i]);
  };
  const int chunks = (tasks + kChunk - 1) / kChunk;
  if (chunks > 1) {
    f32x4 ya[kBmvXStaged], yb[kBmvXStaged];
    for (int c = 0; c < chunks; c += 2) {
      load_chunk(ya, yb, c + 1);
      quantize_chunk(xa, xb, c);
      load_chunk(xa, xb, c + 2);
      if (c + 1 < chunks) quantize_chunk(ya, yb, c + 1);
    }
  } else {
    quantize_chunk(xa, xb, 0);
  }
  if (tid == 0) *reinterpret_cast<lds_u32x4*>(codes + 8 * stride) = u32x4{0u, 0u, 0u, 0u};
  __syncthreads();

  if constexpr (TYPE == QK_TYPE_Q4_K) {
    bmv_stream<TYPE, P, 1>(sh, lc, L, stride, groups_max, codes, xs, xss, xf, sums, buf, start);
  } else {
    if (M > 4)
      bmv_stream<TYPE, P, 2>(sh, lc, L, stride, groups_max, codes, xs, xss, xf, sums, buf, start);
    else
      bmv_stream<TYPE, P, 1>(sh, lc, L, stride, groups_max, codes, xs, xss, xf, sums, buf, start);
  }
  __syncthreads();

  // row totals: runs added in order; one thread per (activation row, row)
  const int nrows = sh.nrows, R = sh.ranges;
  for (int idx = tid; idx < nrows * M; idx += 64 * kBmvWaves) {
    const int m = idx / nrows, row = idx - m * nrows;
    const lds_f32* pa = sums + ((row >> 4) * 16 + (row & 15)) * R * 8 + m;
    float a = 0.0f;
    for (int rr = 0; rr < R; ++rr) a += pa[rr * 8];
    if constexpr (MODE == 0) {
      yout[static_cast<int64_t>(m) * rows_seg + sh.r0 + row] = a;
    } else {
      const lds_f32* pb = pa + groups_max * 16 * R * 8;
      float b = 0.0f;
      for (int rr = 0; rr < R; ++rr) b += pb[rr * 8];
      float* dst = p.h + static_cast<int64_t>(m) * rows_seg + sh.r0 + row;
      const float hv = (a / (1.0f + expf(-a))) * b;
      if (p.hq != nullptr)  // read back by the workgroup that completes the block
        __hip_atomic_store(dst, hv, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      else
        *dst = hv;
    }
  }
  if constexpr (MODE == 1) {
    if (p.hq != nullptr) bmv_close_blocks(p, sh, rows_seg, lds_raw);
  }
}

// TYPE: QK_TYPE_Q4_K or QK_TYPE_Q6_K for launches of one type, 0 for a mixed
// launch (each workgroup takes its segment's type).
template <int TYPE, int MODE>
__global__ __launch_bounds__(64 * kBmvWaves) void bmv_kernel(const BmvParams p) {
  extern __shared__ __align__(16) unsigned char lds_raw[];
#pragma unroll
  for (int j = 0; j < kMaxSegments; ++j)
    asm volatile("" ::"s"(p.seg[j].w), "s"(p.seg[j].y), "s"(p.seg[j].rows), "s"(p.seg[j].type),
                 "s"(p.seg[j].wg_begin), "s"(p.seg[j].per), "s"(p.seg[j].rem), "s"(p.seg[j].pad));
  asm volatile("" ::"s"(p.x), "s"(p.h), "s"(p.hq), "s"(p.arrive), "s"(p.M), "s"(p.K), "s"(p.S), "s"(p.nseg),
               "s"(p.stride), "s"(p.ranges), "s"(p.groups_max), "s"(p.pad));
  __builtin_amdgcn_sched_barrier(0);
  const int wg = static_cast<int>(blockIdx.x), nseg = p.nseg;
  const int j = (nseg > 1 && wg >= p.seg[1].wg_begin) + (nseg > 2 && wg >= p.seg[2].wg_begin) +
                (nseg > 3 && wg >= p.seg[3].wg_begin);
  auto pick = [j](auto f0, auto f1, auto f2, auto f3) {
    return j == 0 ? f0 : j == 1 ? f1 : j == 2 ? f2 : f3;
  };
  const int type = pick(p.seg[0].type, p.seg[1].type, p.seg[2].type, p.seg[3].type);
  const int rows = pick(p.seg[0].rows, p.seg[1].rows, p.seg[2].rows, p.seg[3].rows);
  const int g = wg - pick(p.seg[0].wg_begin, p.seg[1].wg_begin, p.seg[2].wg_begin, p.seg[3].wg_begin);
  const int per = pick(p.seg[0].per, p.seg[1].per, p.seg[2].per, p.seg[3].per);
  const int rem = pick(p.seg[0].rem, p.seg[1].rem, p.seg[2].rem, p.seg[3].rem);
  float* yout = pick(p.seg[0].y, p.seg[1].y, p.seg[2].y, p.seg[3].y);

  BmvShare sh;
  sh.w[0] = pick(p.seg[0].w, p.seg[1].w, p.seg[2].w, p.seg[3].w);
  sh.w[1] = MODE == 1 ? p.seg[1].w : sh.w[0];
  sh.r0 = g * per + min(g, rem);
  sh.nrows = per + (g < rem ? 1 : 0);
  sh.per = per;
  sh.rem = rem;
  sh.groups = (sh.nrows + 15) >> 4;
  sh.S = p.S;
  sh.ranges = p.ranges;
  sh.run_q = p.S / p.ranges;
  sh.run_r = p.S - sh.run_q * p.ranges;
  if constexpr (TYPE == 0) {
    if (type == QK_TYPE_Q4_K) {
      sh.row_bytes = p.S * kQ4KBytes;
      bmv_body<QK_TYPE_Q4_K, MODE, kBmvP4>(p, sh, rows, yout, p.groups_max, lds_raw);
    } else {
      sh.row_bytes = p.S * kQ6KBytes;
      bmv_body<QK_TYPE_Q6_K, MODE, kBmvP6Mixed>(p, sh, rows, yout, p.groups_max, lds_raw);
    }
  } else {
    sh.row_bytes = p.S * (TYPE == QK_TYPE_Q4_K ? kQ4KBytes : kQ6KBytes);
    bmv_body<TYPE, MODE, TYPE == QK_TYPE_Q4_K ? kBmvP4 : kBmvP6>(p, sh, rows, yout, p.groups_max, lds_raw);
  }
}

using BmvKernel = void (*)(BmvParams);

BmvKernel bmv_kernel_for(int type, int mode) {
  if (mode == 1) {
    if (type == QK_TYPE_Q4_K) return &bmv_kernel<QK_TYPE_Q4_K, 1>;
    if (type == QK_TYPE_Q6_K) return &bmv_kernel<QK_TYPE_Q6_K, 1>;
    return nullptr;
  }
  if (type == QK_TYPE_Q4_K) return &bmv_kernel<QK_TYPE_Q4_K, 0>;
  if (type == QK_TYPE_Q6_K) return &bmv_kernel<QK_TYPE_Q6_K, 0>;
  return &bmv_kernel<0, 0>;
}

int superblock_bytes(int type) { return type == QK_TYPE_Q4_K ? kQ4KBytes : kQ6KBytes; }

}  // namespace

// Tiles on the busiest wave when `rows` rows (parts of them each) are cut
// into groups of 16 and each group's S superblocks into `ranges` runs, and
// the units are dealt to kBmvWaves waves in contiguous blocks.
int64_t bmv_wave_tiles(int64_t rows, int parts, int S, int ranges) {
  if (rows <= 0) return 0;
  const int64_t groups = (rows + 15) / 16;
  const int64_t units = parts * groups * ranges;
  const int64_t per_wave = (units + kBmvWaves - 1) / kBmvWaves;
  return per_wave * ((S + ranges - 1) / ranges);
}

// The workgroup counts and run split of a launch (shared with the CPU index
// model of the tests through the same rules). Returns false when the shape
// does not fit this kernel's LDS plan.
bool bmv_plan(const MatvecParams& p, int mode, int cus, int max_lds, int (&count)[kMaxSegments],
              int& ranges, int& groups_max, int& lds) {
  const int nseg = mode == 1 ? 1 : p.nseg;
  const int parts = mode == 1 ? 2 : 1;
  if (nseg > cus) return false;
  double bytes[kMaxSegments] = {0.0}, total = 0.0;
  for (int j = 0; j < nseg; ++j) {
    bytes[j] = static_cast<double>(p.seg[j].rows) * p.S * superblock_bytes(p.seg[j].type) * parts;
    total += bytes[j];
  }
  int sum = 0;
  for (int j = 0; j < nseg; ++j) {
    count[j] = std::clamp(static_cast<int>(cus * bytes[j] / total + 0.5), 1, p.seg[j].rows);
    sum += count[j];
  }
  while (sum > cus) {  // trim the segment with the most workgroups
    int big = 0;
    for (int j = 1; j < nseg; ++j)
      if (count[j] > count[big]) big = j;
    --count[big];
    --sum;
  }
  const int stride = p.K + 16;
  groups_max = 0;
  for (int j = 0; j < nseg; ++j) {
    const int rows_max = (p.seg[j].rows + count[j] - 1) / count[j];
    groups_max = std::max(groups_max, (rows_max + 15) / 16);
  }
  // runs per group: the fewest tiles on the busiest wave of any workgroup,
  // then the fewest units (each unit ends with a lane reduction)
  ranges = 0;
  int64_t best = INT64_MAX;
  for (int r = 1; r <= p.S; ++r) {
    if (bmv_lds_bytes(p.K, stride, parts, groups_max, r) > max_lds) break;
    int64_t tiles = 0, units = 0;
    for (int j = 0; j < nseg; ++j) {
      const int per = p.seg[j].rows / count[j];
      for (int n : {per, per + 1}) {
        tiles = std::max(tiles, bmv_wave_tiles(n, parts, p.S, r));
        units = std::max<int64_t>(units, (parts * ((n + 15) / 16) * r + kBmvWaves - 1) / kBmvWaves);
      }
    }
    const int64_t cost = 8 * tiles + units;
    if (cost < best) {
      best = cost;
      ranges = r;
    }
  }
  if (ranges == 0) return false;
  lds = bmv_lds_bytes(p.K, stride, parts, groups_max, ranges);
  return true;
}

hipError_t launch_bmv(const MatvecParams& p, int mode, hipStream_t stream, bool& launched) {
  launched = false;
  // The gate/up launch (mode 1) only, for now: measured on MI355X at M = 8
  // against the streaming and batched whole-share kernels, gate/up 14.7 us
  // against 19.1; the one-matrix and q/k/v launches are not yet faster here.
  if (p.x == nullptr || p.M < 2 || p.M > 8 || mode != 1) return hipSuccess;
  if (p.K > (INT32_MAX - 64) / 8) return hipSuccess;
  int cus = 0, max_lds = 0;
  hipError_t e = device_limits(cus, max_lds);
  if (e != hipSuccess) return e;
  int count[kMaxSegments] = {0}, ranges = 0, groups_max = 0, lds = 0;
  if (!bmv_plan(p, mode, cus, max_lds, count, ranges, groups_max, lds)) return hipSuccess;
  if (p.hq != nullptr) {  // Q8(h) in the launch: a quad per (block, activation row) of a share
    const int64_t rows_max = (p.seg[0].rows + count[0] - 1) / count[0];
    const int64_t blocks = (rows_max + 30) / 32 + 1;  // blocks a run of rows_max rows can touch
    if (p.seg[0].rows % 32 != 0 || blocks > kBmvMaxCloseBlocks || 4 * blocks * p.M > 64 * kBmvWaves ||
        p.arrive == nullptr)
      return hipSuccess;
  }

  const int nseg = mode == 1 ? 1 : p.nseg;
  BmvParams bp{};
  bp.x = p.x;
  bp.h = p.h;
  bp.hq = p.hq;
  bp.arrive = p.hq != nullptr ? p.arrive : nullptr;
  bp.M = p.M;
  bp.K = p.K;
  bp.S = p.S;
  bp.nseg = nseg;
  bp.stride = p.K + 16;
  bp.ranges = ranges;
  bp.groups_max = groups_max;
  bool q4 = false, q6 = false;
  int begin = 0;
  for (int j = 0; j < nseg; ++j) {
    bp.seg[j] = {p.seg[j].w, p.seg[j].y, p.seg[j].rows, p.seg[j].type, begin,
                 p.seg[j].rows / count[j], p.seg[j].rows % count[j], 0};
    (p.seg[j].type == QK_TYPE_Q4_K ? q4 : q6) = true;
    begin += count[j];
  }
  if (mode == 1) bp.seg[1] = {p.seg[1].w, nullptr, p.seg[1].rows, p.seg[1].type, 0, 0, 0, 0};
  const int type = q4 && q6 ? 0 : q4 ? QK_TYPE_Q4_K : QK_TYPE_Q6_K;
  const BmvKernel fn = bmv_kernel_for(type, mode);
  if (!fn) return hipSuccess;
  e = allow_lds(reinterpret_cast<const void*>(fn), lds);
  if (e != hipSuccess) return e;
  note("bmv_kernel", begin, type, mode, ranges, groups_max, p.hq != nullptr);
  hipLaunchKernelGGL(fn, dim3(static_cast<uint32_t>(begin)), dim3(64 * kBmvWaves),
                     static_cast<size_t>(lds), stream, bp);
  launched = true;
  return hipGetLastError();
}

}  // namespace qk
