// Internal launchers shared by the kernel translation units and the C-ABI
// layer. Every launcher enqueues on `stream` and returns the hipError_t of
// the launch; shapes are validated by the caller (abi.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "qk_abi.h"

namespace qk {

constexpr int kMaxSegments = 4;

// Records the last product kernel a launcher enqueued on this thread: its
// name, up to 6 template values and the grid (qk_last_launch formats it;
// tests and the bench print it to show which instantiation ran).
void note_launch(const char* kernel, int nvalues, const int* values, int64_t grid);
template <typename... T>
inline void note(const char* kernel, int64_t grid, T... values) {
  const int v[] = {static_cast<int>(values)..., 0};
  note_launch(kernel, static_cast<int>(sizeof...(T)), v, grid);
}

// Sets this thread's qk_last_error() message (with the HIP error's text
// unless it is hipSuccess) and returns `code`.
int set_error(int code, const char* message, hipError_t error);

// One weight matrix of a mat-vec launch (rows = N, y is [M x N]).
struct MatvecSegment {
  const uint8_t* w;
  float* y;
  int32_t rows;
  int32_t type;
  int32_t row_begin;  // first row of this segment in the launch's row space (set by launch_matvec)
  int32_t pad;
};

// Kernel arguments of the streaming mat-vec. Exactly one of x (fp32, quantised
// in the prologue) and q8 (pre-quantised blocks) is non-null.
struct MatvecParams {
  const float* x;
  const qk_q8_block* q8;
  float* h;  // FFN mode: SiLU(gate)*up output [M x N]
  int32_t M, K, S, nseg;
  int32_t rows_total;           // rows of all segments (FFN mode: of gate)
  int32_t split_wg, split_row;  // mixed types: workgroups / rows of the Q4_K part
  int32_t pad;
  const float* norm;            // FFN-with-norm mode (3): RMSNorm scale [K]
  float eps;                    // its epsilon
  int32_t pad2;
  void* argmax_ws;              // argmax mode: ArgmaxWorkspace (argmax.hpp)
  uint32_t* argmax_result;      // argmax mode: index of the largest output
  qk_q8_block* hq;              // FFN mode, batched kernel only: Q8(h) [M][N/32] formed in the launch
  uint32_t* arrive;             // with hq: per-block arrival counters [N/32], zero between launches
  MatvecSegment seg[kMaxSegments];
};

// mode 0: y_j = x . W_j^T for every segment (M <= 8);
// mode 1: seg[0] = gate, seg[1] = up, h = SiLU(x . gate^T) * (x . up^T);
// mode 2: M = 1, one segment, y optional, *argmax_result = argmax of y.
hipError_t launch_matvec(MatvecParams p, int mode, hipStream_t stream);

// The whole-share mat-vec for M = 1 (gemv_stream.hip): launched (and
// `launched` set) when every workgroup's share of the weights fits in LDS;
// otherwise nothing is enqueued and launch_matvec uses the streaming kernel.
hipError_t launch_stream_matvec(const MatvecParams& p, int mode, hipStream_t stream, bool& launched);

// The multi-pass whole-share mat-vec (gemv_pass.hip): M = 1, one Q4_K or Q6_K
// matrix, modes 0 and 2, rows up to kPassMaxJ KB; launched (and `launched`
// set) when it takes the shape.
hipError_t launch_pass_matvec(const MatvecParams& p, int mode, hipStream_t stream, bool& launched);

// The whole-share batched mat-vec on the int8 matrix cores (bmv_ws.hip): M =
// 2..8 rows of fp32 activations (modes 0 and 1) or of Q8 blocks (mode 0);
// launched (and `launched` set) when every workgroup's rows fit its phased
// LDS plan.
hipError_t launch_bmv_ws(const MatvecParams& p, int mode, hipStream_t stream, bool& launched);

// The batched mat-vec on the int8 matrix cores (bmv.hip): M = 2..8 rows of
// fp32 activations, the gate/up mode (1); with p.hq and p.arrive it also
// writes Q8(h). Launched (and `launched` set) when the shape fits its LDS
// plan (and, with p.hq, its block-closing step); otherwise nothing is
// enqueued.
hipError_t launch_bmv(const MatvecParams& p, int mode, hipStream_t stream, bool& launched);

// The multi-pass batched mat-vec on the int8 matrix cores (bmv_pass.hip): M =
// 2..8 rows of fp32 activations, mode 0, one matrix tall enough for two
// 16-row groups per wave (the lm_head); launched (and `launched` set) when it
// takes the shape. bmv_pass_plan: superblock columns per pass, 16-byte chunks
// per run and per lane (false when a one-column pass needs more than 8 KB).
hipError_t launch_bmv_pass(const MatvecParams& p, int mode, hipStream_t stream, bool& launched);
bool bmv_pass_plan(int64_t S, int type, int& C, int& cpr, int& J);

// Compute units and LDS bytes per workgroup of the current device (cached).
hipError_t device_limits(int& cus, int& max_lds);
// Sets a kernel's dynamic LDS limit to `lds` bytes (once per kernel and size).
hipError_t allow_lds(const void* fn, int lds);

// The FFN block of one activation row in one launch (ffn_fused.hip): h =
// SiLU(Q8(x') . gate^T) * (Q8(x') . up^T) with x' = x or RMSNorm(x) (norm
// non-null), then y = Q8(h) . down^T; sync is the barrier workspace. Launched
// (and `launched` set) when the shapes fit its one-workgroup-per-CU plan;
// otherwise nothing is enqueued.
struct FfnArgs {
  const float* x;
  const float* norm;
  float eps;
  const void* gate;
  const void* up;
  int gate_up_type;
  const void* down;
  int down_type;
  int64_t K, N;
  float* h;
  float* y;
  void* sync;
};
hipError_t launch_ffn_fused(const FfnArgs& a, hipStream_t stream, bool& launched);
// Bytes of the barrier workspace of launch_ffn_fused.
size_t ffn_sync_bytes();
// Byte offset in the FFN workspace of the word a timed-out grid barrier sets.
size_t ffn_timeout_offset();

// Activation rows one launch_matvec can take for width K (its Q8 blocks live
// in LDS): 8, 4, 2 or 1, or 0 when even one row does not fit.
int matvec_rows_per_launch(int64_t K);

// Activation rows above which matmul runs as the MFMA GEMM instead of the mat-vec.
constexpr int64_t kGemvMaxRows = 8;

// Bytes of device scratch the prefill GEMM needs for M x K activations (their
// fp16 Q8 round trip, row scales, block sums) and, when the launch splits K,
// the partial products of an N-column product of this type; rounded up to 256.
size_t gemm_workspace_bytes(int64_t M, int64_t K, int type, int64_t N);

// A short prompt (at most kGemmShortRows rows) times matrices of at most
// kGemmShortTiles 128-column tiles each: the GEMM forms its activation planes
// itself (no prep launch). A call's matrices either all take this form or all
// take the prep (the GEMM launches below get x, or null and the prepared
// workspace).
constexpr int64_t kGemmShortRows = 32;
constexpr int64_t kGemmShortTiles = 32;
inline bool gemm_short_plan(int64_t M, int64_t N) {
  return M <= kGemmShortRows && (N + 127) / 128 <= kGemmShortTiles;
}

// workspace (>= gemm_workspace_bytes(M, K, ...), 16-byte aligned) = fp16 of
// the Q8 round trip of x[M x K], row scales, block sums (not needed when every
// product of the call takes the short form: `skip`).
hipError_t launch_gemm_prep(const float* x, int64_t M, int64_t K, void* workspace,
                            hipStream_t stream, bool skip = false);

// y[M x N] = x . dequant(W)^T on MFMA, fp32 accumulation, over the prepared
// workspace (M <= kGemmShortRows: over x itself).
hipError_t launch_gemm_core(const float* x, const void* workspace, const void* w, int type, int64_t K,
                            int64_t N, float* y, int64_t M, hipStream_t stream);

// The Q4_K / Q6_K GEMM (gemm_kquant.hip) over the prepared planes: hi (lo
// follows it), row scales and (Q4_K) sub-block sums of the workspace, partial
// products in `partials` (gemm_kq_partial_bytes of them; unused when 0).
// gemm_kq_fits: the shape is within its 32-bit tile and row indices.
bool gemm_kq_fits(int64_t M, int64_t K, int64_t N);
size_t gemm_kq_partial_bytes(int type, int64_t M, int64_t K, int64_t N);
hipError_t launch_gemm_kq(int type, const float* x, const _Float16* hi, const float* row_scale,
                          const void* xsums, const void* w, int64_t K, int64_t N, float* y, int64_t M,
                          float* partials, hipStream_t stream);

// 2..4 weight matrices of width K (either type) on the same prepared
// activations in one launch (attn q, k and v; gate and up): launched (and
// `launched` set) when none needs a split K and all take the combined grid's
// tile shape, else nothing is enqueued. Each output equals its single launch's
// bit for bit.
hipError_t launch_gemm_kq_multi(const float* x, const _Float16* hi, const float* row_scale, const void* xsums,
                                const qk_segment* segments, int count, int64_t K, int64_t M,
                                hipStream_t stream, bool& launched);
hipError_t launch_gemm_core_multi(const float* x, const void* workspace, const qk_segment* segments, int count,
                                  int64_t K, int64_t M, hipStream_t stream, bool& launched);

// Bytes of the argmax workspace (zero-filled once by the caller).
size_t argmax_workspace_bytes();
// Byte offsets in that workspace of the timeout word and of the partial slots.
size_t argmax_timeout_offset();
size_t argmax_slots_bytes();

// *result = argmax of logits[0, count) with the reference's rules.
hipError_t launch_argmax(const float* logits, int64_t count, void* workspace, uint32_t* result,
                         hipStream_t stream);

hipError_t launch_quantize_q8(const float* x, int64_t M, int64_t K, qk_q8_block* q8,
                              hipStream_t stream);

hipError_t launch_dequantize_rows(const void* packed, float* out, int64_t rows, int64_t K,
                                  size_t row_bytes, int type, hipStream_t stream);

// out[rows x width] = RMSNorm of x with per-column scale (src/cuda/rms_norm.cu:6-24).
hipError_t launch_rms_norm(const float* x, const float* scale, float* out, int64_t rows,
                           int64_t width, float eps, hipStream_t stream);

// state[i] += branch[i] for i < count (src/cuda/residual_add.cu:6-9).
hipError_t launch_residual_add(float* state, const float* branch, int64_t count,
                               hipStream_t stream);

hipError_t launch_silu_multiply(const float* gate, const float* up, float* out, int64_t count,
                                hipStream_t stream);

hipError_t launch_synth_superblocks(void* w, int type, int64_t N, int64_t K, uint64_t seed,
                                    float dmax, float dminmax, hipStream_t stream);

hipError_t launch_synth_normal(float* x, int64_t count, uint64_t seed, hipStream_t stream);

}  // namespace qk
