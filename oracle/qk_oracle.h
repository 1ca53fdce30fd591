/*
 * qk_oracle.h — CPU oracle for the Q4_K/Q6_K dequantize-matmul path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker: it is linked or
 * loaded only by tests/, by __graft_entry__.smoke() and by bench.py's
 * cpu_baseline leg. The product (the HIP library and the C++ host layer)
 * never calls it, and nothing here is a fallback for the GPU path.
 *
 * It restates, in plain C, the arithmetic of the reference engine's CPU
 * test oracle and of its GPU kernels:
 *   - superblock dequantisation  src/cuda/embedding.cu:6-59
 *   - Q8 activation quantisation src/cuda/matmul.cu:8-22
 *   - Q8 round trip              src/tests/reference/MatmulReference.hpp:11-29
 *   - reference product (double) src/tests/reference/MatmulReference.hpp:42-64
 *   - integer dp4a decomposition src/cuda/matmul.cu:24-84
 *   - SiLU * up                  src/cuda/silu_multiply.cu:6-12
 *   - argmax (ties -> lowest id) src/cuda/argmax.cu:25-98
 * ggml's to_float (dequantize_row_q4_K / dequantize_row_q6_K; ggml
 * GIT_TAG master, CMakeLists.txt:30-37, not vendored) is the function the
 * reference oracle calls; its arithmetic equals embedding.cu's formula,
 * which is what is restated here.
 *
 * Build with -ffp-contract=off so every float operation rounds as written.
 */
#ifndef QK_ORACLE_H
#define QK_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { QKO_TYPE_Q4_K = 12, QKO_TYPE_Q6_K = 14 };
enum { QKO_Q4K_BYTES = 144, QKO_Q6K_BYTES = 210, QKO_QK = 256 };

/* fp16 <-> fp32 (exact widening incl. subnormals; round-to-nearest-even narrowing). */
float qko_fp16_to_fp32(uint16_t h);
uint16_t qko_fp32_to_fp16(float f);

/* get_scale_min_k4: 6-bit scale/min of sub-block g from the 12-byte field
 * (src/cuda/embedding.cu:20-23, src/cuda/matmul.cu:40-48). */
void qko_get_scale_min_k4(int g, const uint8_t *scales, int *sc, int *m);

/* One row of K weights (K % 256 == 0) -> fp32 (src/cuda/embedding.cu:6-59). */
void qko_dequantize_row_q4k(const uint8_t *row, float *out, int64_t K);
void qko_dequantize_row_q6k(const uint8_t *row, float *out, int64_t K);
/* kernels::dequantize_embeddings semantics (src/cuda/embedding.cu:65-84). 0 ok, 2 bad type. */
int qko_dequantize_rows(const void *packed, float *out, int64_t rows, int64_t K,
                        size_t row_bytes, int type);

/* Q8 quantisation of activations in blocks of 32 (count % 32 == 0):
 * codes[i] = amax==0 ? 0 : (int8)roundf((x/amax)*127), scales[i/32] = amax/127. */
void qko_quantize_q8(const float *x, int8_t *codes, float *scales, int64_t count);
/* round(x/amax*127) * (amax/127) per block of 32 (MatmulReference.hpp:11-29). */
void qko_q8_roundtrip(const float *x, float *out, int64_t count);

/* y[m*N+n] = sum_k double(q8rt(x)[m,k]) * double(w_n[k]); x is [M x K] row-major fp32,
 * w is N rows of K/256 superblocks. threads <= 0 means all processors.
 * Returns 0, 1 (bad shape) or 2 (bad type). (MatmulReference.hpp:42-64) */
int qko_reference_product(const float *x, const void *w, int type, int64_t K, int64_t N,
                          int64_t M, double *y, int threads);
/* Same product accumulated in fp32 (the "fp32 accumulation" CPU variant). */
int qko_reference_product_f32(const float *x, const void *w, int type, int64_t K,
                              int64_t N, int64_t M, float *y, int threads);
/* The reference GPU kernel's decomposition: Q8 codes, per-lane integer dot of 8
 * weights, fp32 epilogue s_g*(d*sc*dot - dmin*m*sum) (src/cuda/matmul.cu:24-84). */
int qko_integer_product(const float *x, const void *w, int type, int64_t K, int64_t N,
                        int64_t M, float *y);

/* out = gate/(1+exp(-gate)) * up (src/cuda/silu_multiply.cu:6-12). */
void qko_silu_multiply(const float *gate, const float *up, float *out, int64_t count);
void qko_rms_norm(const float *x, const float *scale, float *out, int64_t rows, int64_t width,
                  float eps);
/* Index of the largest value; ties resolve to the lowest index (src/cuda/argmax.cu:25-98). */
int64_t qko_argmax(const float *v, int64_t count);

/* ---- Synthetic data: counter-based SplitMix64 --------------------------------
 * word(seed, i) is the i-th output of SplitMix64 seeded with `seed`:
 *   mix64(seed + (i + 1) * 0x9E3779B97F4A7C15).
 * Q4_K superblock b (row-major over N x K/256) draws words 20b..20b+19:
 *   d = fp16(u24(w0) * dmax), dmin = fp16(u24(w1) * dminmax),
 *   scales[0..11] = bytes 0..11 of w2,w3 (little-endian), qs[0..127] = w4..w19.
 * Q6_K superblock b draws words 27b..27b+26:
 *   ql = w0..w15, qh = w16..w23, scales[i] = int8((byte_i & 127) - 64) from w24,w25,
 *   d = fp16(u24(w26) * dmax).
 * Normal activation i draws words 2i, 2i+1: Box-Muller in double,
 *   u1 = 1 - u24(w_2i), u2 = u24(w_2i+1), z = sqrt(-2 ln u1) cos(2 pi u2).
 * u24(w) = (w >> 40) * 2^-24. */
uint64_t qko_mix64(uint64_t z);
uint64_t qko_word(uint64_t seed, uint64_t i);
void qko_synth_superblocks(void *w, int type, int64_t N, int64_t K, uint64_t seed,
                           float dmax, float dminmax);
void qko_synth_normal(float *x, int64_t count, uint64_t seed);

#ifdef __cplusplus
}
#endif
#endif
