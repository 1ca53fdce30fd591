// extern "C" entry points of libqk_hip.so (declared in include/qk_abi.h).
// Validation mirrors kernels::matmul (src/cuda/matmul.cu:132-137) and
// kernels::dequantize_embeddings (src/cuda/embedding.cu:67-70); launch errors
// map to the codes the C++ layer turns into the reference's exceptions
// (include/Kernels.hpp:28-32).
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <algorithm>
#include <string>
#include <cstdint>
#include <climits>

#include "qk_abi.h"
#include "qk_launch.hpp"

namespace {

thread_local std::string g_last_error;

struct LaunchNote {
  const char* kernel = nullptr;
  int nvalues = 0;
  int values[6] = {0};
  int64_t grid = 0;
};
thread_local LaunchNote g_launch;
thread_local std::string g_launch_text;

int fail(int code, const std::string& message) {
  g_last_error = message;
  return code;
}

int hip_fail(hipError_t error, const char* what) {
  const int code = error == hipErrorOutOfMemory ? QK_ERR_OUT_OF_MEMORY : QK_ERR_RUNTIME;
  return fail(code, std::string(what) + ": " + hipGetErrorString(error));
}

bool supported_type(int type) { return type == QK_TYPE_Q4_K || type == QK_TYPE_Q6_K; }

size_t superblock_bytes(int type) {
  return type == QK_TYPE_Q4_K ? 144u : type == QK_TYPE_Q6_K ? 210u : 0u;
}

// The kernels index a row's activations and superblocks in 32 bits.
constexpr int64_t kMaxK = int64_t{1} << 30;

// src/cuda/matmul.cu:132-137 (type, K > 0, K % 256 == 0, N > 0), plus the
// launch-grid bound on rows the reference shares (grid.y = rows) and the
// kernels' 32-bit width bound.
int validate_matmul(int type, int64_t K, int64_t N, int64_t M) {
  if (!supported_type(type))
    return fail(QK_ERR_UNSUPPORTED_TYPE, "matmul supports Q4_K and Q6_K weights only");
  if (K <= 0 || K % 256 != 0 || N <= 0 || N > (int64_t{1} << 31) - 64)
    return fail(QK_ERR_INVALID_ARGUMENT, "Invalid matmul weight dimensions");
  if (K > kMaxK) return fail(QK_ERR_INVALID_ARGUMENT, "Invalid matmul weight dimensions: K exceeds 2^30");
  if (M < 0) return fail(QK_ERR_INVALID_ARGUMENT, "matmul rows must be >= 0");
  return QK_OK;
}

hipStream_t as_stream(qk_stream_t s) { return static_cast<hipStream_t>(s); }

int validate_segment(const qk_segment& sg) {
  if (!supported_type(sg.type))
    return fail(QK_ERR_UNSUPPORTED_TYPE, "matmul supports Q4_K and Q6_K weights only");
  if (sg.N <= 0 || sg.N > (int64_t{1} << 31) - 64)
    return fail(QK_ERR_INVALID_ARGUMENT, "Invalid matmul weight dimensions");
  return QK_OK;
}

// The kernels read Q4_K superblocks in aligned 16-byte pieces and Q6_K ones
// from the dword boundary at or below each field, so the tensor base must be
// 16- (Q4_K) or 4-byte (Q6_K) aligned; device allocations and GGUF tensor
// data (32-byte alignment) always are.
int validate_weight_pointer(const void* w, int type) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(w);
  if (a % (type == QK_TYPE_Q4_K ? 16 : 4) != 0)
    return fail(QK_ERR_INVALID_ARGUMENT,
                type == QK_TYPE_Q4_K ? "Q4_K weights must be 16-byte aligned"
                                     : "Q6_K weights must be 4-byte aligned");
  return QK_OK;
}

// Runs the streaming mat-vec over M activation rows, up to 8 per launch (fewer
// when K is so wide that 8 rows of Q8 blocks do not fit in LDS).
int run_matvec(qk::MatvecParams base, int64_t M, int64_t K, int mode, hipStream_t stream) {
  const int chunk = qk::matvec_rows_per_launch(K);
  if (chunk <= 0) return fail(QK_ERR_INVALID_ARGUMENT, "matmul width K exceeds the LDS capacity");
  base.K = static_cast<int32_t>(K);
  base.S = static_cast<int32_t>(K / 256);
  for (int64_t m0 = 0; m0 < M; m0 += chunk) {
    qk::MatvecParams p = base;
    p.M = static_cast<int32_t>(std::min<int64_t>(chunk, M - m0));
    if (p.x) p.x += m0 * K;
    else p.q8 += m0 * (K / 32);
    for (int j = 0; j < p.nseg; ++j)
      if (p.seg[j].y) p.seg[j].y += m0 * p.seg[j].rows;
    if (p.h) p.h += m0 * p.seg[0].rows;
    const hipError_t error = qk::launch_matvec(p, mode, stream);
    if (error != hipSuccess) return hip_fail(error, "matmul launch failed");
  }
  return QK_OK;
}

int validate_argmax_output(const uint32_t* result, const void* workspace, size_t workspace_bytes) {
  if (!result) return fail(QK_ERR_INVALID_ARGUMENT, "argmax result pointer must be non-null");
  if (!workspace || workspace_bytes < qk::argmax_workspace_bytes() ||
      reinterpret_cast<uintptr_t>(workspace) % 8 != 0)
    return fail(QK_ERR_INVALID_ARGUMENT,
                "argmax workspace must be 8-byte aligned and hold qk_argmax_workspace_size() bytes");
  return QK_OK;
}

qk::MatvecParams params_for(const float* x, const qk_q8_block* q8) {
  qk::MatvecParams p{};
  p.x = x;
  p.q8 = q8;
  return p;
}

int run_single(const float* x, const qk_q8_block* q8, const void* w, int type, int64_t K,
               int64_t N, float* y, int64_t M, hipStream_t stream) {
  const int status = validate_weight_pointer(w, type);
  if (status != QK_OK) return status;
  qk::MatvecParams p = params_for(x, q8);
  p.nseg = 1;
  p.seg[0] = {static_cast<const uint8_t*>(w), y, static_cast<int32_t>(N), type, 0, 0};
  return run_matvec(p, M, K, 0, stream);
}

// Prefill path (M > 8 rows): activation prep once, then one MFMA GEMM per
// weight matrix. Without a caller workspace the fp16 activation scratch is
// allocated stream-ordered for the call, as the reference allocates its Q8
// workspace per call (src/cuda/matmul.cu:143-145).
int run_gemm(const float* x, int64_t M, int64_t K, const qk_segment* segments, int count,
             void* workspace, size_t workspace_bytes, hipStream_t stream) {
  for (int j = 0; j < count; ++j) {
    const int status = validate_weight_pointer(segments[j].w, segments[j].type);
    if (status != QK_OK) return status;
    const int64_t m_tiles = (M + 127) / 128, n_tiles = (segments[j].N + 63) / 64;
    if (M > (int64_t{1} << 31) - 128 || m_tiles * n_tiles > (int64_t{1} << 31) - 1)
      return fail(QK_ERR_INVALID_ARGUMENT, "matmul rows x columns exceed the launch grid");
  }
  size_t need = 0;  // the largest of the segments' needs (they run one after another)
  for (int j = 0; j < count; ++j)
    need = std::max(need, qk::gemm_workspace_bytes(M, K, segments[j].type, segments[j].N));
  void* scratch = workspace;
  if (scratch) {
    if (workspace_bytes < need) return fail(QK_ERR_INVALID_ARGUMENT, "matmul workspace too small");
    if (reinterpret_cast<uintptr_t>(scratch) % 16 != 0)
      return fail(QK_ERR_INVALID_ARGUMENT, "matmul workspace must be 16-byte aligned");
  } else {
    const hipError_t error = hipMallocAsync(&scratch, need, stream);
    if (error != hipSuccess) return hip_fail(error, "matmul workspace allocation failed");
  }
  // short prompt against narrow matrices: the GEMM forms its planes from x
  bool short_form = true;
  for (int j = 0; j < count; ++j) short_form = short_form && qk::gemm_short_plan(M, segments[j].N);
  hipError_t error = qk::launch_gemm_prep(x, M, K, scratch, stream, short_form);
  const float* x_short = short_form ? x : nullptr;
  // every matrix in one launch when they share its tile plan (attn q, k and v:
  // one grid of 768 tiles at M = 512 instead of 640 + 128); otherwise two of
  // one type together where they can, the rest one launch each
  bool all = false;
  if (error == hipSuccess && count > 1)
    error = qk::launch_gemm_core_multi(x_short, scratch, segments, count, K, M, stream, all);
  for (int j = 0; j < count && error == hipSuccess && !all; ++j) {
    if (j + 1 < count && segments[j + 1].type == segments[j].type) {
      bool launched = false;
      error = qk::launch_gemm_core_multi(x_short, scratch, segments + j, 2, K, M, stream, launched);
      if (error != hipSuccess) break;
      if (launched) {
        ++j;
        continue;
      }
    }
    error = qk::launch_gemm_core(x_short, scratch, segments[j].w, segments[j].type, K, segments[j].N,
                                 segments[j].y, M, stream);
  }
  if (!workspace) (void)hipFreeAsync(scratch, stream);
  return error == hipSuccess ? QK_OK : hip_fail(error, "matmul launch failed");
}

int run_gemm_single(const float* x, const void* w, int type, int64_t K, int64_t N, float* y,
                    int64_t M, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  const qk_segment segment{w, type, N, y};
  return run_gemm(x, M, K, &segment, 1, workspace, workspace_bytes, stream);
}

}  // namespace

namespace qk {

int set_error(int code, const char* message, hipError_t error) {
  return error == hipSuccess ? fail(code, message) : hip_fail(error, message);
}

void note_launch(const char* kernel, int nvalues, const int* values, int64_t grid) {
  g_launch.kernel = kernel;
  g_launch.nvalues = std::min(nvalues, 6);
  for (int i = 0; i < g_launch.nvalues; ++i) g_launch.values[i] = values[i];
  g_launch.grid = grid;
}

}  // namespace qk

extern "C" {

const char* qk_last_error(void) { return g_last_error.c_str(); }

const char* qk_last_launch(void) {
  if (!g_launch.kernel) return "";
  std::string text = g_launch.kernel;
  text += '<';
  for (int i = 0; i < g_launch.nvalues; ++i) {
    if (i) text += ',';
    text += std::to_string(g_launch.values[i]);
  }
  text += "> grid=" + std::to_string(g_launch.grid);
  g_launch_text = text;
  return g_launch_text.c_str();
}

int qk_version(void) { return 200; }

size_t qk_matmul_workspace_size(int type, int64_t K, int64_t N, int64_t M) {
  if (!supported_type(type) || K <= 0 || K % 256 != 0 || K > kMaxK || N <= 0 ||
      M <= qk::kGemvMaxRows)
    return 0;
  return qk::gemm_workspace_bytes(M, K, type, N);
}

int qk_matmul(const float* x, const void* w, int type, int64_t K, int64_t N, float* y, int64_t M,
              qk_stream_t stream) {
  const int status = validate_matmul(type, K, N, M);
  if (status != QK_OK) return status;
  if (M == 0) return QK_OK;
  if (!x || !w || !y) return fail(QK_ERR_INVALID_ARGUMENT, "matmul pointers must be non-null");
  if (M > qk::kGemvMaxRows)
    return run_gemm_single(x, w, type, K, N, y, M, nullptr, 0, as_stream(stream));
  return run_single(x, nullptr, w, type, K, N, y, M, as_stream(stream));
}

int qk_matmul_ws(const float* x, const void* w, int type, int64_t K, int64_t N, float* y,
                 int64_t M, void* workspace, size_t workspace_bytes, qk_stream_t stream) {
  const int status = validate_matmul(type, K, N, M);
  if (status != QK_OK) return status;
  if (M == 0) return QK_OK;
  if (!x || !w || !y) return fail(QK_ERR_INVALID_ARGUMENT, "matmul pointers must be non-null");
  if (M <= qk::kGemvMaxRows) return run_single(x, nullptr, w, type, K, N, y, M, as_stream(stream));
  if (!workspace) return fail(QK_ERR_INVALID_ARGUMENT, "matmul workspace must be non-null");
  return run_gemm_single(x, w, type, K, N, y, M, workspace, workspace_bytes, as_stream(stream));
}

int qk_quantize_q8(const float* x, int64_t M, int64_t K, qk_q8_block* q8, qk_stream_t stream) {
  if (M < 0 || K <= 0 || K % 32 != 0)
    return fail(QK_ERR_INVALID_ARGUMENT, "quantize needs M >= 0 and K a positive multiple of 32");
  if (M == 0) return QK_OK;
  if (!x || !q8) return fail(QK_ERR_INVALID_ARGUMENT, "quantize pointers must be non-null");
  if (reinterpret_cast<uintptr_t>(q8) % 16 != 0)
    return fail(QK_ERR_INVALID_ARGUMENT, "Q8 blocks must be 16-byte aligned");
  const hipError_t error = qk::launch_quantize_q8(x, M, K, q8, as_stream(stream));
  return error == hipSuccess ? QK_OK : hip_fail(error, "quantize launch failed");
}

int qk_matmul_q8(const qk_q8_block* q8, const void* w, int type, int64_t K, int64_t N, float* y,
                 int64_t M, qk_stream_t stream) {
  const int status = validate_matmul(type, K, N, M);
  if (status != QK_OK) return status;
  if (M == 0) return QK_OK;
  if (!q8 || !w || !y) return fail(QK_ERR_INVALID_ARGUMENT, "matmul pointers must be non-null");
  if (reinterpret_cast<uintptr_t>(q8) % 16 != 0)
    return fail(QK_ERR_INVALID_ARGUMENT, "Q8 blocks must be 16-byte aligned");
  return run_single(nullptr, q8, w, type, K, N, y, M, as_stream(stream));
}

namespace {

// Prefill FFN (M > 8): gate and up through the GEMM (one launch for both
// where no split K is needed) into scratch, then SiLU(gate) * up into h. The
// scratch (gate and up outputs, then the GEMM workspace) is the caller's
// workspace when given, else allocated stream-ordered for the call.
size_t ffn_gemm_bytes(int type, int64_t K, int64_t N, int64_t M) {
  const size_t gu = (2 * static_cast<size_t>(M) * static_cast<size_t>(N) * sizeof(float) + 255) & ~size_t{255};
  return gu + qk::gemm_workspace_bytes(M, K, type, N);
}

int run_ffn_gemm(const float* x, const void* gate, const void* up, int type, int64_t K, int64_t N,
                 float* h, int64_t M, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  const size_t need = ffn_gemm_bytes(type, K, N, M);
  void* scratch = workspace;
  if (scratch) {
    if (workspace_bytes < need) return fail(QK_ERR_INVALID_ARGUMENT, "ffn workspace too small");
    if (reinterpret_cast<uintptr_t>(scratch) % 16 != 0)
      return fail(QK_ERR_INVALID_ARGUMENT, "ffn workspace must be 16-byte aligned");
  } else {
    const hipError_t error = hipMallocAsync(&scratch, need, stream);
    if (error != hipSuccess) return hip_fail(error, "ffn scratch allocation failed");
  }
  float* gu = static_cast<float*>(scratch);
  const size_t gu_bytes = need - qk::gemm_workspace_bytes(M, K, type, N);
  const qk_segment segments[2] = {{gate, type, N, gu}, {up, type, N, gu + M * N}};
  int status = run_gemm(x, M, K, segments, 2, static_cast<char*>(scratch) + gu_bytes, need - gu_bytes,
                        stream);
  if (status == QK_OK) {
    const hipError_t error = qk::launch_silu_multiply(gu, gu + M * N, h, M * N, stream);
    if (error != hipSuccess) status = hip_fail(error, "silu_multiply launch failed");
  }
  if (!workspace) (void)hipFreeAsync(scratch, stream);
  return status;
}

int ffn_gate_up(const float* x, const void* gate, const void* up, int type, int64_t K, int64_t N,
                float* h, int64_t M, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  const int status = validate_matmul(type, K, N, M);
  if (status != QK_OK) return status;
  if (M == 0) return QK_OK;
  if (!x || !gate || !up || !h) return fail(QK_ERR_INVALID_ARGUMENT, "ffn pointers must be non-null");
  for (const void* w : {gate, up}) {
    const int status = validate_weight_pointer(w, type);
    if (status != QK_OK) return status;
  }
  if (M > qk::kGemvMaxRows)
    return run_ffn_gemm(x, gate, up, type, K, N, h, M, workspace, workspace_bytes, stream);
  qk::MatvecParams p = params_for(x, nullptr);
  p.nseg = 2;
  p.h = h;
  p.seg[0] = {static_cast<const uint8_t*>(gate), nullptr, static_cast<int32_t>(N), type, 0, 0};
  p.seg[1] = {static_cast<const uint8_t*>(up), nullptr, static_cast<int32_t>(N), type, 0, 0};
  return run_matvec(p, M, K, 1, stream);
}

// Largest workspace of the segments (they run one after another on one prep).
size_t segments_gemm_bytes(int64_t M, int64_t K, const qk_segment* segments, int count) {
  size_t need = 0;
  for (int j = 0; j < count; ++j)
    need = std::max(need, qk::gemm_workspace_bytes(M, K, segments[j].type, segments[j].N));
  return need;
}

int matmul_segments(const float* x, int64_t M, int64_t K, const qk_segment* segments, int count,
                    void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (count < 1 || count > qk::kMaxSegments || !segments)
    return fail(QK_ERR_INVALID_ARGUMENT, "segment count must be in [1, 4]");
  if (K <= 0 || K % 256 != 0) return fail(QK_ERR_INVALID_ARGUMENT, "Invalid matmul weight dimensions");
  if (K > kMaxK) return fail(QK_ERR_INVALID_ARGUMENT, "Invalid matmul weight dimensions: K exceeds 2^30");
  if (M < 0) return fail(QK_ERR_INVALID_ARGUMENT, "matmul rows must be >= 0");
  for (int j = 0; j < count; ++j) {
    const int status = validate_segment(segments[j]);
    if (status != QK_OK) return status;
  }
  if (M == 0) return QK_OK;
  if (!x) return fail(QK_ERR_INVALID_ARGUMENT, "matmul pointers must be non-null");
  for (int j = 0; j < count; ++j)
    if (!segments[j].w || !segments[j].y)
      return fail(QK_ERR_INVALID_ARGUMENT, "matmul pointers must be non-null");
  if (M > qk::kGemvMaxRows) return run_gemm(x, M, K, segments, count, workspace, workspace_bytes, stream);
  qk::MatvecParams p = params_for(x, nullptr);
  p.nseg = count;
  for (int j = 0; j < count; ++j) {
    const int status = validate_weight_pointer(segments[j].w, segments[j].type);
    if (status != QK_OK) return status;
    p.seg[j] = {static_cast<const uint8_t*>(segments[j].w), segments[j].y,
                static_cast<int32_t>(segments[j].N), segments[j].type, 0, 0};
  }
  return run_matvec(p, M, K, 0, stream);
}

}  // namespace

int qk_matmul_segments(const float* x, int64_t M, int64_t K, const qk_segment* segments, int count,
                       qk_stream_t stream) {
  return matmul_segments(x, M, K, segments, count, nullptr, 0, as_stream(stream));
}

size_t qk_matmul_segments_workspace_size(int64_t M, int64_t K, const qk_segment* segments, int count) {
  if (!segments || count < 1 || count > qk::kMaxSegments || K <= 0 || K % 256 != 0 || K > kMaxK ||
      M <= qk::kGemvMaxRows)
    return 0;
  for (int j = 0; j < count; ++j)
    if (!supported_type(segments[j].type) || segments[j].N <= 0) return 0;
  return segments_gemm_bytes(M, K, segments, count);
}

int qk_matmul_segments_ws(const float* x, int64_t M, int64_t K, const qk_segment* segments, int count,
                          void* workspace, size_t workspace_bytes, qk_stream_t stream) {
  if (M > qk::kGemvMaxRows && !workspace)
    return fail(QK_ERR_INVALID_ARGUMENT, "matmul workspace must be non-null");
  return matmul_segments(x, M, K, segments, count, workspace, workspace_bytes, as_stream(stream));
}

int qk_ffn_gate_up(const float* x, const void* gate, const void* up, int type, int64_t K, int64_t N,
                   float* h, int64_t M, qk_stream_t stream) {
  return ffn_gate_up(x, gate, up, type, K, N, h, M, nullptr, 0, as_stream(stream));
}

size_t qk_ffn_gate_up_workspace_size(int type, int64_t K, int64_t N, int64_t M) {
  if (!supported_type(type) || K <= 0 || K % 256 != 0 || K > kMaxK || N <= 0 ||
      N > (int64_t{1} << 31) - 64 || M <= qk::kGemvMaxRows)
    return 0;
  return ffn_gemm_bytes(type, K, N, M);
}

int qk_ffn_gate_up_ws(const float* x, const void* gate, const void* up, int type, int64_t K, int64_t N,
                      float* h, int64_t M, void* workspace, size_t workspace_bytes, qk_stream_t stream) {
  if (M > qk::kGemvMaxRows && !workspace)
    return fail(QK_ERR_INVALID_ARGUMENT, "ffn workspace must be non-null");
  return ffn_gate_up(x, gate, up, type, K, N, h, M, workspace, workspace_bytes, as_stream(stream));
}

int qk_ffn_gate_up_norm(const float* x, const float* norm, float eps, const void* gate, const void* up,
                        int type, int64_t K, int64_t N, float* h, int64_t M, qk_stream_t stream) {
  const int status = validate_matmul(type, K, N, M);
  if (status != QK_OK) return status;
  if (M == 0) return QK_OK;  // src/cuda/rms_norm.cu:31
  if (!(eps > 0.0f))        // src/cuda/rms_norm.cu:32
    return fail(QK_ERR_INVALID_ARGUMENT, "RMSNorm requires a positive epsilon");
  if (!x || !norm || !gate || !up || !h)
    return fail(QK_ERR_INVALID_ARGUMENT, "ffn pointers must be non-null");
  for (const void* w : {gate, up}) {
    const int status = validate_weight_pointer(w, type);
    if (status != QK_OK) return status;
  }
  qk::MatvecParams p = params_for(x, nullptr);
  p.nseg = 2;
  p.h = h;
  p.seg[0] = {static_cast<const uint8_t*>(gate), nullptr, static_cast<int32_t>(N), type, 0, 0};
  p.seg[1] = {static_cast<const uint8_t*>(up), nullptr, static_cast<int32_t>(N), type, 0, 0};
  const hipStream_t s = as_stream(stream);
  if (M == 1) {  // the norm folded into the whole-share kernel's prologue
    p.M = 1;
    p.K = static_cast<int32_t>(K);
    p.S = static_cast<int32_t>(K / 256);
    p.norm = norm;
    p.eps = eps;
    bool launched = false;
    const hipError_t error = qk::launch_stream_matvec(p, 3, s, launched);
    if (error != hipSuccess) return hip_fail(error, "matmul launch failed");
    if (launched) return QK_OK;
  }
  // Otherwise the norm runs on its own into stream-ordered scratch, then the
  // fused gate/up product.
  float* normalized = nullptr;
  hipError_t error = hipMallocAsync(reinterpret_cast<void**>(&normalized),
                                    static_cast<size_t>(M * K) * sizeof(float), s);
  if (error != hipSuccess) return hip_fail(error, "RMSNorm scratch allocation failed");
  error = qk::launch_rms_norm(x, norm, normalized, M, K, eps, s);
  int result = error == hipSuccess ? QK_OK : hip_fail(error, "RMSNorm launch failed");
  if (result == QK_OK) result = qk_ffn_gate_up(normalized, gate, up, type, K, N, h, M, stream);
  (void)hipFreeAsync(normalized, s);
  return result;
}

// qk_ffn workspace: the grid-barrier words, then (M = 2..8) Q8(h) and the
// normalised rows, so the batched block allocates nothing and quantises h once
// instead of in every CU of the down launch.
constexpr size_t kFfnQ8Bytes = size_t{160} << 10;    // Q8 image of h, M*N/32 blocks
constexpr size_t kFfnNormBytes = size_t{512} << 10;  // RMSNorm(x) rows, M*K floats
constexpr size_t kFfnArriveBytes = size_t{8} << 10;  // Q8(h) block arrival counters, N/32 words

size_t qk_ffn_workspace_size(void) {
  return qk::ffn_sync_bytes() + kFfnQ8Bytes + kFfnNormBytes + kFfnArriveBytes;
}

int qk_ffn(const float* x, const float* norm, float eps, const void* gate, const void* up,
           int gate_up_type, const void* down, int down_type, int64_t K, int64_t N, float* h, float* y,
           int64_t M, void* workspace, size_t workspace_bytes, qk_stream_t stream) {
  int status = validate_matmul(gate_up_type, K, N, M);  // gate/up: N rows of width K
  if (status != QK_OK) return status;
  status = validate_matmul(down_type, N, K, M);  // down: K rows of width N
  if (status != QK_OK) return status;
  if (M == 0) return QK_OK;
  if (norm && !(eps > 0.0f))  // src/cuda/rms_norm.cu:32
    return fail(QK_ERR_INVALID_ARGUMENT, "RMSNorm requires a positive epsilon");
  if (!x || !gate || !up || !down || !h || !y)
    return fail(QK_ERR_INVALID_ARGUMENT, "ffn pointers must be non-null");
  if (!workspace || workspace_bytes < qk_ffn_workspace_size() ||
      reinterpret_cast<uintptr_t>(workspace) % 256 != 0)
    return fail(QK_ERR_INVALID_ARGUMENT,
                "ffn workspace must be 256-byte aligned and hold qk_ffn_workspace_size() bytes");
  for (const void* w : {gate, up}) {
    status = validate_weight_pointer(w, gate_up_type);
    if (status != QK_OK) return status;
  }
  status = validate_weight_pointer(down, down_type);
  if (status != QK_OK) return status;
  const hipStream_t s = as_stream(stream);
  if (M == 1) {
    const qk::FfnArgs a{x, norm, eps, gate, up, gate_up_type, down, down_type, K, N, h, y, workspace};
    bool launched = false;
    const hipError_t error = qk::launch_ffn_fused(a, s, launched);
    if (error != hipSuccess) return hip_fail(error, "ffn launch failed");
    if (launched) return QK_OK;
  }
  // M = 2..8 with a full workspace: RMSNorm rows and Q8(h) in the workspace;
  // gate/up with h quantised once (in the gate/up launch when the batched
  // kernel takes it, else by its own launch), the down mat-vec on the Q8
  // blocks.
  const size_t q8_bytes = static_cast<size_t>(M) * static_cast<size_t>(N / 32) * sizeof(qk_q8_block);
  const size_t norm_bytes = norm ? static_cast<size_t>(M * K) * sizeof(float) : 0;
  if (M >= 2 && M <= 8 && q8_bytes <= kFfnQ8Bytes && norm_bytes <= kFfnNormBytes &&
      qk::matvec_rows_per_launch(N) >= M) {
    char* base = static_cast<char*>(workspace) + qk::ffn_sync_bytes();
    qk_q8_block* hq = reinterpret_cast<qk_q8_block*>(base);
    const float* xin = x;
    if (norm) {
      float* normalized = reinterpret_cast<float*>(base + kFfnQ8Bytes);
      const hipError_t error = qk::launch_rms_norm(x, norm, normalized, M, K, eps, s);
      if (error != hipSuccess) return hip_fail(error, "RMSNorm launch failed");
      xin = normalized;
    }
    qk::MatvecParams p = params_for(xin, nullptr);
    p.M = static_cast<int32_t>(M);
    p.K = static_cast<int32_t>(K);
    p.S = static_cast<int32_t>(K / 256);
    p.nseg = 2;
    p.h = h;
    p.seg[0] = {static_cast<const uint8_t*>(gate), nullptr, static_cast<int32_t>(N), gate_up_type, 0, 0};
    p.seg[1] = {static_cast<const uint8_t*>(up), nullptr, static_cast<int32_t>(N), gate_up_type, 0, 0};
    if (static_cast<size_t>(N / 32) * sizeof(uint32_t) <= kFfnArriveBytes) {
      p.hq = hq;
      p.arrive = reinterpret_cast<uint32_t*>(base + kFfnQ8Bytes + kFfnNormBytes);
    }
    bool fused_q8 = false;
    hipError_t error = p.hq ? qk::launch_bmv(p, 1, s, fused_q8) : hipSuccess;
    if (error != hipSuccess) return hip_fail(error, "ffn gate/up launch failed");
    if (!fused_q8) {
      status = qk_ffn_gate_up(xin, gate, up, gate_up_type, K, N, h, M, stream);
      if (status != QK_OK) return status;
      error = qk::launch_quantize_q8(h, M, N, hq, s);
      if (error != hipSuccess) return hip_fail(error, "quantize launch failed");
    }
    return run_single(nullptr, hq, down, down_type, N, K, y, M, s);
  }
  // Otherwise: the fused gate/up (with the norm when given), then down.
  status = norm ? qk_ffn_gate_up_norm(x, norm, eps, gate, up, gate_up_type, K, N, h, M, stream)
                : qk_ffn_gate_up(x, gate, up, gate_up_type, K, N, h, M, stream);
  if (status != QK_OK) return status;
  return qk_matmul(h, down, down_type, N, K, y, M, stream);
}

int qk_ffn_workspace_check(void* workspace, qk_stream_t stream) {
  if (!workspace) return fail(QK_ERR_INVALID_ARGUMENT, "ffn workspace must be non-null");
  uint32_t flag = 0;
  const size_t at = qk::ffn_timeout_offset();
  hipError_t error = hipMemcpyAsync(&flag, static_cast<char*>(workspace) + at, sizeof(flag),
                                    hipMemcpyDeviceToHost, as_stream(stream));
  if (error == hipSuccess) error = hipStreamSynchronize(as_stream(stream));
  if (error != hipSuccess) return hip_fail(error, "ffn workspace read failed");
  if (flag == 0) return QK_OK;
  const uint32_t zero = 0;
  error = hipMemcpyAsync(static_cast<char*>(workspace) + at, &zero, sizeof(zero), hipMemcpyHostToDevice,
                         as_stream(stream));
  if (error == hipSuccess) error = hipStreamSynchronize(as_stream(stream));
  if (error != hipSuccess) return hip_fail(error, "ffn workspace reset failed");
  return fail(QK_ERR_RUNTIME,
              "ffn grid barrier timed out: not every workgroup was resident; outputs of that call are invalid");
}

size_t qk_argmax_workspace_size(void) { return qk::argmax_workspace_bytes(); }

int qk_argmax_workspace_check(void* workspace, qk_stream_t stream) {
  if (!workspace) return fail(QK_ERR_INVALID_ARGUMENT, "argmax workspace must be non-null");
  uint32_t flag = 0;
  char* base = static_cast<char*>(workspace);
  hipError_t error = hipMemcpyAsync(&flag, base + qk::argmax_timeout_offset(), sizeof(flag),
                                    hipMemcpyDeviceToHost, as_stream(stream));
  if (error == hipSuccess) error = hipStreamSynchronize(as_stream(stream));
  if (error != hipSuccess) return hip_fail(error, "argmax workspace read failed");
  if (flag == 0) return QK_OK;
  // The late partial a timed-out collector skipped may have landed in its
  // slot after the collector cleared it: the stream is idle now, so clear
  // every slot and the word for the next call.
  error = hipMemsetAsync(base, 0, qk::argmax_slots_bytes(), as_stream(stream));
  const uint32_t zero = 0;
  if (error == hipSuccess)
    error = hipMemcpyAsync(base + qk::argmax_timeout_offset(), &zero, sizeof(zero), hipMemcpyHostToDevice,
                           as_stream(stream));
  if (error == hipSuccess) error = hipStreamSynchronize(as_stream(stream));
  if (error != hipSuccess) return hip_fail(error, "argmax workspace reset failed");
  return fail(QK_ERR_RUNTIME,
              "argmax collector timed out waiting for a workgroup's candidate; the index of that call is invalid");
}

int qk_argmax(const float* logits, int64_t count, uint32_t* result, void* workspace,
              size_t workspace_bytes, qk_stream_t stream) {
  // src/cuda/argmax.cu:73-74
  if (!logits || count <= 0 || count > int64_t{UINT32_MAX})
    return fail(QK_ERR_INVALID_ARGUMENT, "Invalid argmax input");
  const int status = validate_argmax_output(result, workspace, workspace_bytes);
  if (status != QK_OK) return status;
  const hipError_t error = qk::launch_argmax(logits, count, workspace, result, as_stream(stream));
  return error == hipSuccess ? QK_OK : hip_fail(error, "argmax launch failed");
}

int qk_matmul_argmax(const float* x, const void* w, int type, int64_t K, int64_t N, float* logits,
                     uint32_t* result, void* workspace, size_t workspace_bytes, qk_stream_t stream) {
  int status = validate_matmul(type, K, N, 1);
  if (status != QK_OK) return status;
  if (!x || !w) return fail(QK_ERR_INVALID_ARGUMENT, "matmul pointers must be non-null");
  status = validate_argmax_output(result, workspace, workspace_bytes);
  if (status != QK_OK) return status;
  status = validate_weight_pointer(w, type);
  if (status != QK_OK) return status;
  qk::MatvecParams p = params_for(x, nullptr);
  p.nseg = 1;
  p.seg[0] = {static_cast<const uint8_t*>(w), logits, static_cast<int32_t>(N), type, 0, 0};
  p.argmax_ws = workspace;
  p.argmax_result = result;
  return run_matvec(p, 1, K, 2, as_stream(stream));
}

int qk_dequantize_rows(const void* packed, float* out, int64_t rows, int64_t K, size_t row_bytes,
                       int type, qk_stream_t stream) {
  if (rows == 0) return QK_OK;  // src/cuda/embedding.cu:67
  if (!supported_type(type))
    return fail(QK_ERR_UNSUPPORTED_TYPE, "Unsupported embedding storage type");
  if (rows < 0 || K <= 0 || K % 256 != 0 ||
      row_bytes < static_cast<size_t>(K / 256) * superblock_bytes(type))
    return fail(QK_ERR_INVALID_ARGUMENT, "Invalid dequantize dimensions");
  if (!packed || !out) return fail(QK_ERR_INVALID_ARGUMENT, "dequantize pointers must be non-null");
  const hipError_t error =
      qk::launch_dequantize_rows(packed, out, rows, K, row_bytes, type, as_stream(stream));
  return error == hipSuccess ? QK_OK : hip_fail(error, "dequantize launch failed");
}

int qk_rms_norm(const float* x, const float* scale, float* out, int64_t rows, int64_t width,
                float eps, qk_stream_t stream) {
  if (rows < 0) return fail(QK_ERR_INVALID_ARGUMENT, "RMSNorm rows must be >= 0");
  if (rows == 0) return QK_OK;  // src/cuda/rms_norm.cu:31
  if (width <= 0 || width > INT32_MAX || !(eps > 0.0f) || rows > UINT32_MAX)  // :32-34
    return fail(QK_ERR_INVALID_ARGUMENT,
                "RMSNorm requires an F32 scale matching the row width and positive epsilon");
  if (!x || !scale || !out) return fail(QK_ERR_INVALID_ARGUMENT, "RMSNorm pointers must be non-null");
  const hipError_t error = qk::launch_rms_norm(x, scale, out, rows, width, eps, as_stream(stream));
  return error == hipSuccess ? QK_OK : hip_fail(error, "RMSNorm launch failed");
}

int qk_residual_add(float* state, const float* branch, int64_t count, qk_stream_t stream) {
  if (count < 0) return fail(QK_ERR_INVALID_ARGUMENT, "count must be >= 0");
  if (count == 0) return QK_OK;  // src/cuda/residual_add.cu:16
  if (!state || !branch) return fail(QK_ERR_INVALID_ARGUMENT, "pointers must be non-null");
  const hipError_t error = qk::launch_residual_add(state, branch, count, as_stream(stream));
  return error == hipSuccess ? QK_OK : hip_fail(error, "residual_add launch failed");
}

int qk_check_launch(void) {
  const hipError_t error = hipGetLastError();
  return error == hipSuccess ? QK_OK : fail(QK_ERR_RUNTIME, hipGetErrorString(error));
}

int qk_silu_multiply(const float* gate, const float* up, float* out, int64_t count,
                     qk_stream_t stream) {
  if (count < 0) return fail(QK_ERR_INVALID_ARGUMENT, "count must be >= 0");
  if (count == 0) return QK_OK;  // src/cuda/silu_multiply.cu:20
  if (!gate || !up || !out) return fail(QK_ERR_INVALID_ARGUMENT, "pointers must be non-null");
  const hipError_t error = qk::launch_silu_multiply(gate, up, out, count, as_stream(stream));
  return error == hipSuccess ? QK_OK : hip_fail(error, "silu_multiply launch failed");
}

// ------------------------------------------------------------ memory shims --

int qk_malloc(void** ptr, size_t bytes) {
  if (!ptr) return fail(QK_ERR_INVALID_ARGUMENT, "null output pointer");
  *ptr = nullptr;
  if (bytes == 0) return QK_OK;  // src/Weight.cpp:27: empty buffers hold nullptr
  const hipError_t error = hipMalloc(ptr, bytes);
  return error == hipSuccess ? QK_OK : hip_fail(error, "hipMalloc failed");
}

int qk_free(void* ptr) {
  if (!ptr) return QK_OK;
  const hipError_t error = hipFree(ptr);
  return error == hipSuccess ? QK_OK : hip_fail(error, "hipFree failed");
}

int qk_malloc_async(void** ptr, size_t bytes, qk_stream_t stream) {
  if (!ptr) return fail(QK_ERR_INVALID_ARGUMENT, "null output pointer");
  *ptr = nullptr;
  if (bytes == 0) return QK_OK;
  const hipError_t error = hipMallocAsync(ptr, bytes, as_stream(stream));
  return error == hipSuccess ? QK_OK : hip_fail(error, "hipMallocAsync failed");
}

int qk_free_async(void* ptr, qk_stream_t stream) {
  if (!ptr) return QK_OK;
  const hipError_t error = hipFreeAsync(ptr, as_stream(stream));
  return error == hipSuccess ? QK_OK : hip_fail(error, "hipFreeAsync failed");
}

int qk_memcpy_h2d(void* dst, const void* src, size_t bytes, qk_stream_t stream) {
  if (bytes == 0) return QK_OK;
  hipError_t error = hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, as_stream(stream));
  if (error == hipSuccess) error = hipStreamSynchronize(as_stream(stream));
  return error == hipSuccess ? QK_OK : hip_fail(error, "host-to-device copy failed");
}

int qk_memcpy_d2h(void* dst, const void* src, size_t bytes, qk_stream_t stream) {
  if (bytes == 0) return QK_OK;
  hipError_t error = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, as_stream(stream));
  if (error == hipSuccess) error = hipStreamSynchronize(as_stream(stream));
  return error == hipSuccess ? QK_OK : hip_fail(error, "device-to-host copy failed");
}

int qk_memcpy_d2d_async(void* dst, const void* src, size_t bytes, qk_stream_t stream) {
  if (bytes == 0) return QK_OK;
  const hipError_t error =
      hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, as_stream(stream));
  return error == hipSuccess ? QK_OK : hip_fail(error, "device-to-device copy failed");
}

int qk_memset_async(void* ptr, int value, size_t bytes, qk_stream_t stream) {
  if (bytes == 0) return QK_OK;
  const hipError_t error = hipMemsetAsync(ptr, value, bytes, as_stream(stream));
  return error == hipSuccess ? QK_OK : hip_fail(error, "memset failed");
}

int qk_stream_create(qk_stream_t* stream) {
  if (!stream) return fail(QK_ERR_INVALID_ARGUMENT, "null output pointer");
  hipStream_t s = nullptr;
  const hipError_t error = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
  if (error != hipSuccess) return hip_fail(error, "stream creation failed");
  *stream = s;
  return QK_OK;
}

int qk_stream_destroy(qk_stream_t stream) {
  if (!stream) return QK_OK;
  const hipError_t error = hipStreamDestroy(as_stream(stream));
  return error == hipSuccess ? QK_OK : hip_fail(error, "stream destruction failed");
}

int qk_stream_synchronize(qk_stream_t stream) {
  const hipError_t error = hipStreamSynchronize(as_stream(stream));
  return error == hipSuccess ? QK_OK : hip_fail(error, "stream synchronize failed");
}

int qk_stream_query(qk_stream_t stream, int* ready) {
  if (!ready) return fail(QK_ERR_INVALID_ARGUMENT, "null output pointer");
  const hipError_t error = hipStreamQuery(as_stream(stream));
  if (error == hipErrorNotReady) {
    *ready = 0;
    return QK_OK;
  }
  if (error != hipSuccess) return hip_fail(error, "stream query failed");
  *ready = 1;
  return QK_OK;
}

int qk_device_synchronize(void) {
  const hipError_t error = hipDeviceSynchronize();
  return error == hipSuccess ? QK_OK : hip_fail(error, "device synchronize failed");
}

int qk_device_count(int* count) {
  if (!count) return fail(QK_ERR_INVALID_ARGUMENT, "null output pointer");
  *count = 0;
  const hipError_t error = hipGetDeviceCount(count);
  if (error == hipErrorNoDevice) {
    *count = 0;
    return QK_OK;
  }
  return error == hipSuccess ? QK_OK : hip_fail(error, "device count failed");
}

int qk_set_device(int device) {
  const hipError_t error = hipSetDevice(device);
  return error == hipSuccess ? QK_OK : hip_fail(error, "set device failed");
}

int qk_device_info(char* name, size_t name_len, int* compute_units, char* arch, size_t arch_len) {
  int device = 0;
  hipError_t error = hipGetDevice(&device);
  if (error != hipSuccess) return hip_fail(error, "get device failed");
  hipDeviceProp_t prop;
  error = hipGetDeviceProperties(&prop, device);
  if (error != hipSuccess) return hip_fail(error, "device properties failed");
  if (name && name_len) std::snprintf(name, name_len, "%s", prop.name);
  if (arch && arch_len) std::snprintf(arch, arch_len, "%s", prop.gcnArchName);
  if (compute_units) *compute_units = prop.multiProcessorCount;
  return QK_OK;
}

int qk_event_create(qk_event_t* event) {
  if (!event) return fail(QK_ERR_INVALID_ARGUMENT, "null output pointer");
  hipEvent_t e = nullptr;
  const hipError_t error = hipEventCreate(&e);
  if (error != hipSuccess) return hip_fail(error, "event creation failed");
  *event = e;
  return QK_OK;
}

int qk_event_destroy(qk_event_t event) {
  if (!event) return QK_OK;
  const hipError_t error = hipEventDestroy(static_cast<hipEvent_t>(event));
  return error == hipSuccess ? QK_OK : hip_fail(error, "event destruction failed");
}

int qk_event_record(qk_event_t event, qk_stream_t stream) {
  const hipError_t error = hipEventRecord(static_cast<hipEvent_t>(event), as_stream(stream));
  return error == hipSuccess ? QK_OK : hip_fail(error, "event record failed");
}

int qk_event_synchronize(qk_event_t event) {
  const hipError_t error = hipEventSynchronize(static_cast<hipEvent_t>(event));
  return error == hipSuccess ? QK_OK : hip_fail(error, "event synchronize failed");
}

int qk_event_elapsed_ms(float* ms, qk_event_t start, qk_event_t end) {
  if (!ms) return fail(QK_ERR_INVALID_ARGUMENT, "null output pointer");
  const hipError_t error =
      hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(end));
  return error == hipSuccess ? QK_OK : hip_fail(error, "event elapsed time failed");
}

// ------------------------------------------------------------------ graphs --

int qk_stream_begin_capture(qk_stream_t stream) {
  if (!stream) return fail(QK_ERR_INVALID_ARGUMENT, "capture needs a non-null stream");
  const hipError_t error = hipStreamBeginCapture(as_stream(stream), hipStreamCaptureModeThreadLocal);
  return error == hipSuccess ? QK_OK : hip_fail(error, "begin capture failed");
}

int qk_stream_end_capture(qk_stream_t stream, qk_graph_t* graph) {
  if (!stream || !graph) return fail(QK_ERR_INVALID_ARGUMENT, "capture needs a stream and an output");
  *graph = nullptr;
  hipGraph_t captured = nullptr;
  hipError_t error = hipStreamEndCapture(as_stream(stream), &captured);
  if (error != hipSuccess) return hip_fail(error, "end capture failed");
  hipGraphExec_t exec = nullptr;
  error = hipGraphInstantiate(&exec, captured, nullptr, nullptr, 0);
  (void)hipGraphDestroy(captured);
  if (error != hipSuccess) return hip_fail(error, "graph instantiation failed");
  *graph = exec;
  return QK_OK;
}

int qk_graph_launch(qk_graph_t graph, qk_stream_t stream) {
  if (!graph) return fail(QK_ERR_INVALID_ARGUMENT, "null graph");
  const hipError_t error = hipGraphLaunch(static_cast<hipGraphExec_t>(graph), as_stream(stream));
  return error == hipSuccess ? QK_OK : hip_fail(error, "graph launch failed");
}

int qk_graph_destroy(qk_graph_t graph) {
  if (!graph) return QK_OK;
  const hipError_t error = hipGraphExecDestroy(static_cast<hipGraphExec_t>(graph));
  return error == hipSuccess ? QK_OK : hip_fail(error, "graph destruction failed");
}

// -------------------------------------------------------------- synthetic --

int qk_synth_superblocks(void* w, int type, int64_t N, int64_t K, uint64_t seed, float dmax,
                         float dminmax, qk_stream_t stream) {
  if (!supported_type(type)) return fail(QK_ERR_UNSUPPORTED_TYPE, "synth supports Q4_K and Q6_K");
  if (N < 0 || K <= 0 || K % 256 != 0) return fail(QK_ERR_INVALID_ARGUMENT, "Invalid synth shape");
  if (N == 0) return QK_OK;
  if (!w) return fail(QK_ERR_INVALID_ARGUMENT, "synth pointer must be non-null");
  const hipError_t error =
      qk::launch_synth_superblocks(w, type, N, K, seed, dmax, dminmax, as_stream(stream));
  return error == hipSuccess ? QK_OK : hip_fail(error, "synth launch failed");
}

int qk_synth_normal(float* x, int64_t count, uint64_t seed, qk_stream_t stream) {
  if (count < 0) return fail(QK_ERR_INVALID_ARGUMENT, "count must be >= 0");
  if (count == 0) return QK_OK;
  if (!x) return fail(QK_ERR_INVALID_ARGUMENT, "synth pointer must be non-null");
  const hipError_t error = qk::launch_synth_normal(x, count, seed, as_stream(stream));
  return error == hipSuccess ? QK_OK : hip_fail(error, "synth launch failed");
}

}  // extern "C"
