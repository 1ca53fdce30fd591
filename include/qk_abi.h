/*
 * qk_abi.h — C-ABI of the MI355X (gfx950) Q4_K/Q6_K dequantize-matmul library
 * (libqk_hip.so). Plain pointers and sizes only: no HIP, CUDA or torch types.
 *
 * Conventions (src/cuda/matmul.cu:130-162, include/Kernels.hpp:9-10):
 *   - x is a device fp32 row-major [M x K] activation matrix.
 *   - w is the raw GGUF tensor bytes on the device: N rows, each K/256
 *     superblocks (Q4_K: 144 bytes, Q6_K: 210 bytes), no repacking.
 *     K = ggml ne[0] (Weight::dimension[0]), N = ne[1] (Weight::dimension[1]).
 *   - y is a device fp32 row-major [M x N] output; it is overwritten.
 *   - every launch is asynchronous on `stream` (NULL = the null stream).
 *   - status: QK_OK, or an error code with a message in qk_last_error()
 *     (thread-local, valid until the next failing call on the same thread).
 */
#ifndef QK_ABI_H
#define QK_ABI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum qk_status {
    QK_OK = 0,
    QK_ERR_INVALID_ARGUMENT = 1, /* std::invalid_argument in the C++ layer */
    QK_ERR_UNSUPPORTED_TYPE = 2, /* std::invalid_argument in the C++ layer */
    QK_ERR_RUNTIME = 3,          /* std::runtime_error in the C++ layer */
    QK_ERR_OUT_OF_MEMORY = 4     /* std::runtime_error in the C++ layer */
};

/* GGUF on-disk tensor type ids (the values of ggml_type). */
enum qk_type { QK_TYPE_F32 = 0, QK_TYPE_F16 = 1, QK_TYPE_Q4_K = 12, QK_TYPE_Q6_K = 14 };

typedef void *qk_stream_t; /* a hipStream_t; NULL is the null stream */
typedef void *qk_event_t;  /* a hipEvent_t */
typedef void *qk_graph_t;  /* an instantiated hipGraphExec_t */

/* Q8 activation block: 32 consecutive activations of one row.
 * codes[i] = amax==0 ? 0 : (int8)roundf((x_i/amax)*127), scale = amax/127
 * (the quantisation of src/cuda/matmul.cu:8-22), plus the sums the
 * superblock dots need: scaled_sum = scale*sum(codes),
 * neg32_sum_lo/hi = -32*sum(codes[0..15]) / -32*sum(codes[16..31]). */
typedef struct qk_q8_block {
    int8_t codes[32];
    float scale;
    float scaled_sum;
    int32_t neg32_sum_lo;
    int32_t neg32_sum_hi;
} qk_q8_block;

/* One weight matrix of a multi-segment mat-vec: N rows of `type` superblocks,
 * output y [M x N]. */
typedef struct qk_segment {
    const void *w;
    int type;
    int64_t N;
    float *y;
} qk_segment;

/* Message of the last failing call on this thread ("" if none). */
const char *qk_last_error(void);
/* The last product kernel launched by a call on this thread, as
 * "name<template values> grid=G" ("" if none); diagnostics only, valid until
 * the next call of qk_last_launch on the same thread. No counterpart in the
 * reference. */
const char *qk_last_launch(void);
/* Library version: major*10000 + minor*100 + patch. */
int qk_version(void);

/* ---------------------------------------------------------------------------
 * Dequantize-matmul (the hot path).
 * ------------------------------------------------------------------------- */

/* y[M x N] = Q8(x)[M x K] . W^T. Replaces kernels::matmul
 * (include/Kernels.hpp:57-61, src/cuda/matmul.cu:130-165). Validation as the
 * reference: type must be Q4_K or Q6_K (else QK_ERR_UNSUPPORTED_TYPE),
 * K > 0, K % 256 == 0, N > 0 (else QK_ERR_INVALID_ARGUMENT); M == 0 returns
 * QK_OK without launching.
 * M <= 8 (decode): one streaming mat-vec launch per 8 rows, Q8 quantisation
 * inside the kernel, integer dot products as the reference; nothing is
 * allocated. M > 8 (prefill): the activations' Q8 round trip, scaled per row
 * by a power of two, is stored as two fp16 planes hi + lo in a stream-ordered
 * scratch buffer (qk_matmul_workspace_size bytes, allocated and freed on
 * `stream` like the reference's per-call workspace) with the planes' 32-value
 * block sums; an MFMA GEMM multiplies them by the weights in fp32 accumulation:
 * Q4_K as the exact fp16 integers sc*q (hi*B + lo*B per step, d and dmin*m
 * applied once per superblock), Q6_K as sc*q = fp16(sc*q) + an exact
 * remainder in {-1, 0, 1} (hi*B_hi + lo*B_hi + hi*B_lo, d once per
 * superblock). K above 2^30 returns QK_ERR_INVALID_ARGUMENT. */
int qk_matmul(const float *x, const void *w, int type, int64_t K, int64_t N, float *y,
              int64_t M, qk_stream_t stream);

/* Workspace bytes qk_matmul_ws needs for this shape (0 for M <= 8 and for
 * shapes qk_matmul rejects). For M > 8 it holds the activation planes
 * (M*K*4 + M*4 bytes, rounded up to 16), their block sums (M*(K/256)*32) and,
 * when the launch plan splits K (few output tiles, deep K), the partial
 * products (splits*M*N*4); the total is rounded up to 256. The split plan is
 * internal: size workspaces with this function, not from the formula. */
size_t qk_matmul_workspace_size(int type, int64_t K, int64_t N, int64_t M);

/* qk_matmul with a caller-owned device workspace (16-byte aligned) of at least
 * qk_matmul_workspace_size() bytes (may be NULL when that is 0); allocates
 * nothing, so it can be captured into a graph at any M. Same results as
 * qk_matmul. */
int qk_matmul_ws(const float *x, const void *w, int type, int64_t K, int64_t N, float *y,
                 int64_t M, void *workspace, size_t workspace_bytes, qk_stream_t stream);

/* Bytes of the device scratch array behind qk_matmul_noalloc (48 MiB: the
 * prefill workspace of every Qwen3-4B projection up to M = 512 fits). */
#define QK_NOALLOC_SCRATCH_BYTES ((size_t)48 << 20)

/* qk_matmul that allocates nothing, for callers that cannot call hipMalloc
 * (code under graph capture, tight serving loops, harnesses that forbid
 * allocation). No counterpart in the reference. Same validation and results
 * as qk_matmul; at M > 8 the prefill workspace is a file-scope device array of
 * QK_NOALLOC_SCRATCH_BYTES per device (held until the process ends), so shapes
 * whose qk_matmul_workspace_size exceeds it return QK_ERR_INVALID_ARGUMENT.
 * All calls on one device share that array: calls that overlap on one device
 * (e.g. on two streams) race. */
int qk_matmul_noalloc(const float *x, const void *w, int type, int64_t K, int64_t N, float *y,
                      int64_t M, qk_stream_t stream);

/* Step 1 of qk_matmul: x[M x K] -> M*K/32 qk_q8_block (K % 32 == 0).
 * Replaces the quantize kernel of src/cuda/matmul.cu:8-22 (+ the sums). */
int qk_quantize_q8(const float *x, int64_t M, int64_t K, qk_q8_block *q8,
                   qk_stream_t stream);

/* Step 2 of qk_matmul: y = q8 . W^T with q8 from qk_quantize_q8.
 * Replaces project<Q4_K/Q6_K> of src/cuda/matmul.cu:86-125. */
int qk_matmul_q8(const qk_q8_block *q8, const void *w, int type, int64_t K, int64_t N,
                 float *y, int64_t M, qk_stream_t stream);

/* Several projections of the same input in one launch: segments[j].y =
 * Q8(x) . W_j^T for j < count (count <= 4; Q4_K and Q6_K may be mixed, all of
 * width K). Replaces the back-to-back kernels::matmul calls on one input,
 * e.g. attn q/k/v (src/Engine.cpp:83-85). Validation per segment as qk_matmul. */
int qk_matmul_segments(const float *x, int64_t M, int64_t K, const qk_segment *segments,
                       int count, qk_stream_t stream);

/* Workspace bytes qk_matmul_segments_ws needs (0 for M <= 8 and for arguments
 * qk_matmul_segments rejects): the largest of the segments' GEMM workspaces
 * (they run one after another on one activation prep). */
size_t qk_matmul_segments_workspace_size(int64_t M, int64_t K, const qk_segment *segments,
                                         int count);

/* qk_matmul_segments with a caller-owned device workspace (16-byte aligned, at
 * least qk_matmul_segments_workspace_size bytes; may be NULL for M <= 8):
 * allocates nothing, so a prefill can be captured into a graph. */
int qk_matmul_segments_ws(const float *x, int64_t M, int64_t K, const qk_segment *segments,
                          int count, void *workspace, size_t workspace_bytes, qk_stream_t stream);

/* h[M x N] = SiLU(Q8(x) . gate^T) * (Q8(x) . up^T), gate and up both `type`
 * with K columns and N rows: one launch for M <= 8; for M > 8 the prefill
 * GEMM (gate and up in one launch) into stream-ordered scratch, then the
 * SiLU kernel. Replaces matmul(gate), matmul(up), silu_multiply
 * (src/Engine.cpp:98-100, src/cuda/silu_multiply.cu:6-12). */
int qk_ffn_gate_up(const float *x, const void *gate, const void *up, int type, int64_t K,
                   int64_t N, float *h, int64_t M, qk_stream_t stream);

/* Workspace bytes qk_ffn_gate_up_ws needs (0 for M <= 8 and for shapes
 * qk_ffn_gate_up rejects): gate and up outputs (2*M*N*4, rounded up to 256)
 * and the GEMM workspace. */
size_t qk_ffn_gate_up_workspace_size(int type, int64_t K, int64_t N, int64_t M);

/* qk_ffn_gate_up with a caller-owned device workspace (16-byte aligned, at
 * least qk_ffn_gate_up_workspace_size bytes; may be NULL for M <= 8):
 * allocates nothing. Same results as qk_ffn_gate_up. */
int qk_ffn_gate_up_ws(const float *x, const void *gate, const void *up, int type, int64_t K,
                      int64_t N, float *h, int64_t M, void *workspace, size_t workspace_bytes,
                      qk_stream_t stream);

/* qk_ffn_gate_up on RMSNorm(x): each row x_m is first replaced by
 * (x_m * rsqrt(mean(x_m^2) + eps)) * norm (norm: K device floats). Replaces
 * rms_norm(ffn_norm) before the FFN (src/Engine.cpp:97-99,
 * src/cuda/rms_norm.cu:6-24,28-36). M = 1: the norm is folded into the one
 * launch and the normalised row never goes to memory; other M: the norm runs
 * first into stream-ordered scratch. eps must be > 0 (QK_ERR_INVALID_ARGUMENT
 * otherwise, as the reference throws); M = 0 does nothing. */
int qk_ffn_gate_up_norm(const float *x, const float *norm, float eps, const void *gate,
                        const void *up, int type, int64_t K, int64_t N, float *h, int64_t M,
                        qk_stream_t stream);

/* Bytes of the workspace qk_ffn needs: its grid-barrier words, then room for
 * Q8(h) (160 KiB), the RMSNorm rows (512 KiB) and the Q8(h) block arrival
 * counters (8 KiB) of the batched M = 2..8 block.
 * The caller zero-fills it once before its first use; every call leaves it
 * ready for the next. Calls that may run concurrently need separate
 * workspaces. */
size_t qk_ffn_workspace_size(void);

/* The FFN block: h[M x N] = SiLU(Q8(x') . gate^T) * (Q8(x') . up^T) and
 * y[M x K] = Q8(h) . down^T, with x' = RMSNorm(x) (scale `norm`: K device
 * floats, eps > 0) or x itself when norm is NULL. gate and up: N rows of K
 * (gate_up_type), down: K rows of N (down_type). Replaces rms_norm(ffn_norm),
 * matmul(gate), matmul(up), silu_multiply, matmul(down) (src/Engine.cpp:97-101).
 * M = 1 with Q4_K gate/up (the Q4_K_M layout) and shapes that fit one
 * workgroup per CU: ONE launch. Phase 1 is the gate/up product (the norm
 * folded in), each workgroup storing its range of h; a grid barrier; phase 2
 * reads h back, quantises it and runs the down rows, whose weights were
 * loaded during phase 1. That launch needs every workgroup resident at once:
 * do not overlap it with other kernels on the device. Its barrier wait is
 * bounded: if it ever times out, the workgroups that gave up write NaN into
 * their y rows, the outputs of that call are invalid, and
 * qk_ffn_workspace_check reports it (an engine that graph-replays decode steps
 * checks after each replay of a step, or at least before it trusts a token).
 * M = 2..8 (when M*N/32 Q8 blocks fit in
 * 160 KiB, M*K norm rows in 512 KiB and M rows of Q8(h) in one down launch):
 * the norm into the workspace, qk_ffn_gate_up with h quantised once into the
 * workspace (in the gate/up launch, by the workgroup that completes each
 * 32-value block, when N/32 counters fit in 8 KiB; else by a launch of its
 * own), then the down mat-vec on those Q8 blocks; nothing is allocated.
 * Other M or shapes: qk_ffn_gate_up(_norm) then qk_matmul on the stream
 * (allocating at M > 8 as they do). Validation
 * as qk_matmul for both weights, plus the workspace (256-byte aligned, at
 * least qk_ffn_workspace_size bytes) and eps when norm is given. */
int qk_ffn(const float *x, const float *norm, float eps, const void *gate, const void *up,
           int gate_up_type, const void *down, int down_type, int64_t K, int64_t N, float *h,
           float *y, int64_t M, void *workspace, size_t workspace_bytes, qk_stream_t stream);

/* Synchronises `stream`, then returns QK_ERR_RUNTIME (and clears the flag) if
 * a qk_ffn call on this workspace timed out in its grid barrier since the
 * last check, else QK_OK. */
int qk_ffn_workspace_check(void *workspace, qk_stream_t stream);

/* Bytes of the workspace qk_argmax / qk_matmul_argmax need. The caller
 * zero-fills it once before its first use (qk_memset_async or hipMemset);
 * every call leaves it ready for the next. Calls that may run concurrently
 * (different streams) need separate workspaces. */
size_t qk_argmax_workspace_size(void);

/* QK_ERR_RUNTIME if an argmax call on this workspace since the last check
 * stopped waiting for a workgroup's candidate (its collector waits at most
 * 0.2 s for each: only a device that could not start a workgroup for that long
 * gets there): the index that call wrote is invalid, and so may be the index
 * of every later call on the workspace until this check, since the late
 * candidate can land in its slot after the collector cleared it and be taken
 * by the next call as its own. The check clears every slot, so the next call
 * is sound again. Synchronizes `stream`. No counterpart in the
 * reference, whose argmax reduces on the host (src/cuda/argmax.cu:89-97); for
 * callers that keep a workspace across calls, as qk_ffn_workspace_check. */
int qk_argmax_workspace_check(void *workspace, qk_stream_t stream);

/* *result (device uint32) = the index of the largest of logits[0, count): the
 * lowest index among equal maxima; NaN and -inf never win; 0xFFFFFFFF if no
 * entry wins. Replaces kernels::argmax (include/Kernels.hpp:77,
 * src/cuda/argmax.cu:71-98) without its blocking copy: the result stays on the
 * device. count in [1, 2^32-1], else QK_ERR_INVALID_ARGUMENT. */
int qk_argmax(const float *logits, int64_t count, uint32_t *result, void *workspace,
              size_t workspace_bytes, qk_stream_t stream);

/* lm_head and argmax in one launch for one activation row: logits[N] =
 * Q8(x)[K] . W^T (written only if logits != NULL) and *result = the argmax of
 * the logits, with qk_argmax's rules. Replaces kernels::matmul + kernels::argmax
 * at src/Engine.cpp:106-111. Validation as qk_matmul with M = 1, plus
 * qk_argmax's result and workspace rules. */
int qk_matmul_argmax(const float *x, const void *w, int type, int64_t K, int64_t N, float *logits,
                     uint32_t *result, void *workspace, size_t workspace_bytes,
                     qk_stream_t stream);

/* Dequantize `rows` rows of K weights (row stride row_bytes) to fp32
 * out[rows x K], bit-identical to the formulas of src/cuda/embedding.cu:6-59.
 * Replaces kernels::dequantize_embeddings (include/Kernels.hpp:74-75,
 * src/cuda/embedding.cu:65-84); rows == 0 returns QK_OK. */
int qk_dequantize_rows(const void *packed, float *out, int64_t rows, int64_t K,
                       size_t row_bytes, int type, qk_stream_t stream);

/* out[rows x width] = (x * rsqrt(mean(x^2) + eps)) * scale per row, scale a
 * device float[width]. Replaces kernels::rms_norm (include/Kernels.hpp:54-55,
 * src/cuda/rms_norm.cu:6-36): rows == 0 returns QK_OK; width <= 0 (or above
 * 2^31-1), eps <= 0 or rows above 2^32-1 give QK_ERR_INVALID_ARGUMENT. */
int qk_rms_norm(const float *x, const float *scale, float *out, int64_t rows, int64_t width,
                float eps, qk_stream_t stream);

/* state[i] += branch[i] for i < count. Replaces kernels::residual_add
 * (include/Kernels.hpp:70, src/cuda/residual_add.cu:6-20); count == 0
 * returns QK_OK. */
int qk_residual_add(float *state, const float *branch, int64_t count, qk_stream_t stream);

/* Status of the last kernel launch on this thread (the HIP runtime's last
 * error, which this call clears): QK_OK or QK_ERR_RUNTIME with the message in
 * qk_last_error(). Replaces the CUDA query of kernels::detail::check_launch
 * (include/Kernels.hpp:28-32) for engine kernels built outside this library. */
int qk_check_launch(void);

/* out = gate/(1+exp(-gate)) * up, elementwise. Replaces kernels::silu_multiply
 * (include/Kernels.hpp:72, src/cuda/silu_multiply.cu:19-23). */
int qk_silu_multiply(const float *gate, const float *up, float *out, int64_t count,
                     qk_stream_t stream);

/* ---------------------------------------------------------------------------
 * Device memory, streams and events. The thin layer the C++ DeviceBuffer
 * (include/Weight.hpp:8-23, src/Weight.cpp:6-51) and stream class
 * (include/Kernels.hpp:38-52, src/cuda/CudaStream.cpp:13-46) sit on.
 * ------------------------------------------------------------------------- */
int qk_malloc(void **ptr, size_t bytes);
int qk_free(void *ptr);
int qk_malloc_async(void **ptr, size_t bytes, qk_stream_t stream);
int qk_free_async(void *ptr, qk_stream_t stream);
/* Host<->device copies are ordered on `stream` and complete before return. */
int qk_memcpy_h2d(void *dst, const void *src, size_t bytes, qk_stream_t stream);
int qk_memcpy_d2h(void *dst, const void *src, size_t bytes, qk_stream_t stream);
int qk_memcpy_d2d_async(void *dst, const void *src, size_t bytes, qk_stream_t stream);
int qk_memset_async(void *ptr, int value, size_t bytes, qk_stream_t stream);
int qk_stream_create(qk_stream_t *stream); /* non-blocking stream */
int qk_stream_destroy(qk_stream_t stream);
int qk_stream_synchronize(qk_stream_t stream);
int qk_stream_query(qk_stream_t stream, int *ready); /* *ready = 1 when idle */
int qk_device_synchronize(void);
int qk_device_count(int *count);
int qk_set_device(int device);
/* Name, compute units and arch of the current device (name_len bytes incl. NUL). */
int qk_device_info(char *name, size_t name_len, int *compute_units, char *arch,
                   size_t arch_len);
int qk_event_create(qk_event_t *event);
int qk_event_destroy(qk_event_t event);
int qk_event_record(qk_event_t event, qk_stream_t stream);
int qk_event_synchronize(qk_event_t event);
int qk_event_elapsed_ms(float *ms, qk_event_t start, qk_event_t end);

/* ---------------------------------------------------------------------------
 * Graph capture of a launch sequence on a non-null stream, replayed with one
 * call (the reference lists CUDA Graphs as future work, README.md:42). No
 * compute entry point records a memset. At M <= 8 none allocates, except
 * qk_ffn_gate_up_norm outside its M = 1 fold; at M > 8 qk_matmul,
 * qk_matmul_segments, qk_ffn_gate_up, qk_ffn_gate_up_norm and qk_ffn allocate
 * their scratch stream-ordered (captured as allocation nodes), while the _ws
 * entry points take a caller workspace and qk_matmul_noalloc uses the
 * library's scratch array: those allocate nothing.
 * ------------------------------------------------------------------------- */
int qk_stream_begin_capture(qk_stream_t stream);
/* Ends the capture and instantiates it; *graph owns the executable graph. */
int qk_stream_end_capture(qk_stream_t stream, qk_graph_t *graph);
int qk_graph_launch(qk_graph_t graph, qk_stream_t stream);
int qk_graph_destroy(qk_graph_t graph);

/* ---------------------------------------------------------------------------
 * Synthetic inputs generated on the device (no host upload). No reference
 * counterpart: the reference tests read the real model file
 * (src/tests/TestModel.hpp.in:3). word(seed, i) is the i-th SplitMix64 output,
 * mix64(seed + (i+1)*0x9E3779B97F4A7C15), and u24(w) = (w >> 40) * 2^-24.
 *   Q4_K superblock b (row-major) uses words 20b..20b+19: d = fp16(u24(w0)*dmax),
 *     dmin = fp16(u24(w1)*dminmax), scales = bytes 0..11 of w2,w3, qs = w4..w19.
 *   Q6_K superblock b uses words 27b..27b+26: ql = w0..w15, qh = w16..w23,
 *     scales[i] = int8((byte_i of w24,w25 & 127) - 64), d = fp16(u24(w26)*dmax).
 *   Normal value i uses words 2i, 2i+1: Box-Muller in double with
 *     u1 = 1 - u24(w_2i), u2 = u24(w_2i+1), z = sqrt(-2 ln u1) cos(2 pi u2).
 * Bytes are little-endian; fp16 rounding is to nearest even.
 * ------------------------------------------------------------------------- */
int qk_synth_superblocks(void *w, int type, int64_t N, int64_t K, uint64_t seed, float dmax,
                         float dminmax, qk_stream_t stream);
int qk_synth_normal(float *x, int64_t count, uint64_t seed, qk_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* QK_ABI_H */
