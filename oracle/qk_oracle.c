/*
 * qk_oracle.c — CPU oracle for the Q4_K/Q6_K dequantize-matmul path.
 *
 * TEST INFRASTRUCTURE ONLY (see qk_oracle.h): the checker for the HIP path,
 * never part of it. Compiled with -O3 -ffp-contract=off -fopenmp.
 *
 * Each function cites the reference file:line whose arithmetic it restates.
 */
#include "qk_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ---------------------------------------------------------------- fp16 --- */

float qko_fp16_to_fp32(uint16_t h)
{
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    const uint32_t exp = (h >> 10) & 0x1Fu;
    const uint32_t man = h & 0x3FFu;
    uint32_t bits;
    if (exp == 0) {
        /* zero or subnormal: man * 2^-24 is exact in fp32 */
        float v = ldexpf((float)man, -24);
        memcpy(&bits, &v, 4);
        bits |= sign;
    } else if (exp == 31) {
        bits = sign | 0x7F800000u | (man << 13);
    } else {
        bits = sign | ((exp - 15 + 127) << 23) | (man << 13);
    }
    float out;
    memcpy(&out, &bits, 4);
    return out;
}

uint16_t qko_fp32_to_fp16(float f)
{
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) /* inf / nan */
        return (uint16_t)(sign | (ax > 0x7F800000u ? 0x7E00u : 0x7C00u));
    if (ax >= 0x477FF000u) /* >= 65520 rounds to infinity */
        return (uint16_t)(sign | 0x7C00u);
    if (ax < 0x38800000u) { /* below 2^-14: fp16 subnormal or zero */
        float a;
        memcpy(&a, &ax, 4);
        const float scaled = a * 16777216.0f; /* exact: a * 2^24 < 2^10 */
        const uint32_t m = (uint32_t)nearbyintf(scaled); /* ties to even */
        return (uint16_t)(sign | m);
    }
    const uint32_t e = (ax >> 23) - 127 + 15;
    const uint32_t man = ax & 0x7FFFFFu;
    uint32_t h = (e << 10) | (man >> 13);
    const uint32_t rem = man & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u)))
        h++;
    return (uint16_t)(sign | h);
}

static float load_fp16(const uint8_t *p)
{
    return qko_fp16_to_fp32((uint16_t)(p[0] | (p[1] << 8)));
}

/* ------------------------------------------------------------- dequant --- */

/* src/cuda/embedding.cu:20-23 (same bits as src/cuda/matmul.cu:40-48). */
void qko_get_scale_min_k4(int g, const uint8_t *scales, int *sc, int *m)
{
    if (g < 4) {
        *sc = scales[g] & 63;
        *m = scales[g + 4] & 63;
    } else {
        *sc = (scales[g + 4] & 15) | ((scales[g - 4] >> 6) << 4);
        *m = (scales[g + 4] >> 4) | ((scales[g] >> 6) << 4);
    }
}

/* src/cuda/embedding.cu:6-32: w = (d*sc)*q - dmin*m, element p of a superblock. */
void qko_dequantize_row_q4k(const uint8_t *row, float *out, int64_t K)
{
    for (int64_t b = 0; b < K / QKO_QK; ++b) {
        const uint8_t *block = row + b * QKO_Q4K_BYTES;
        const float d = load_fp16(block);
        const float dmin = load_fp16(block + 2);
        const uint8_t *scales = block + 4;
        const uint8_t *qs = block + 16;
        for (int p = 0; p < QKO_QK; ++p) {
            const int g = p / 32;
            int sc, m;
            qko_get_scale_min_k4(g, scales, &sc, &m);
            const unsigned q = (qs[(g / 2) * 32 + p % 32] >> ((g % 2) * 4)) & 15u;
            const float ds = d * (float)sc;
            const float dm = dmin * (float)m;
            out[b * QKO_QK + p] = ds * (float)q - dm;
        }
    }
}

/* src/cuda/embedding.cu:34-59: w = (d*sc)*(q-32). */
void qko_dequantize_row_q6k(const uint8_t *row, float *out, int64_t K)
{
    for (int64_t b = 0; b < K / QKO_QK; ++b) {
        const uint8_t *block = row + b * QKO_Q6K_BYTES;
        const uint8_t *ql = block;
        const uint8_t *qh = block + 128;
        const int8_t *scales = (const int8_t *)(block + 192);
        const float d = load_fp16(block + 208);
        for (int p = 0; p < QKO_QK; ++p) {
            const int half = p / 128;
            const int group = (p % 128) / 32;
            const int lane = p % 32;
            const unsigned low = (ql[half * 64 + (group % 2) * 32 + lane] >> (4 * (group / 2))) & 15u;
            const unsigned high = (qh[half * 32 + lane] >> (2 * group)) & 3u;
            const int code = (int)((high << 4) | low) - 32;
            const int scale = scales[p / 16];
            const float ds = d * (float)scale;
            out[b * QKO_QK + p] = ds * (float)code;
        }
    }
}

static int type_bytes(int type)
{
    return type == QKO_TYPE_Q4_K ? QKO_Q4K_BYTES : type == QKO_TYPE_Q6_K ? QKO_Q6K_BYTES : 0;
}

static void dequantize_row(int type, const uint8_t *row, float *out, int64_t K)
{
    if (type == QKO_TYPE_Q4_K)
        qko_dequantize_row_q4k(row, out, K);
    else
        qko_dequantize_row_q6k(row, out, K);
}

/* src/cuda/embedding.cu:65-84 (kernels::dequantize_embeddings). */
int qko_dequantize_rows(const void *packed, float *out, int64_t rows, int64_t K,
                        size_t row_bytes, int type)
{
    if (rows == 0)
        return 0;
    if (type_bytes(type) == 0)
        return 2;
    const uint8_t *base = (const uint8_t *)packed;
    for (int64_t r = 0; r < rows; ++r)
        dequantize_row(type, base + (size_t)r * row_bytes, out + r * K, K);
    return 0;
}

/* ------------------------------------------------------------------ Q8 --- */

/* src/cuda/matmul.cu:8-22 */
void qko_quantize_q8(const float *x, int8_t *codes, float *scales, int64_t count)
{
    for (int64_t begin = 0; begin < count; begin += 32) {
        float maximum = 0.0f;
        for (int i = 0; i < 32; ++i)
            maximum = fmaxf(maximum, fabsf(x[begin + i]));
        scales[begin / 32] = maximum / 127.0f;
        for (int i = 0; i < 32; ++i) {
            const float v = x[begin + i];
            codes[begin + i] = maximum == 0.0f ? 0 : (int8_t)roundf((v / maximum) * 127.0f);
        }
    }
}

/* src/tests/reference/MatmulReference.hpp:11-29 */
void qko_q8_roundtrip(const float *x, float *out, int64_t count)
{
    for (int64_t begin = 0; begin < count; begin += 32) {
        float maximum = 0.0f;
        for (int i = 0; i < 32; ++i) {
            const float a = fabsf(x[begin + i]);
            maximum = maximum < a ? a : maximum; /* std::max(maximum, a) */
        }
        const float scale = maximum / 127.0f;
        for (int i = 0; i < 32; ++i) {
            const float r = roundf(x[begin + i] / maximum * 127.0f);
            out[begin + i] = maximum == 0.0f ? 0.0f : r * scale;
        }
    }
}

/* ------------------------------------------------------------- products --- */

static int check_shape(int type, int64_t K, int64_t N, int64_t M)
{
    if (type_bytes(type) == 0)
        return 2;
    if (K <= 0 || K % QKO_QK != 0 || N <= 0 || M < 0)
        return 1;
    return 0;
}

/* src/tests/reference/MatmulReference.hpp:42-64: every W row decoded once,
 * accumulated in double over k ascending. Rows n are independent, so the
 * OpenMP split over n does not change any output bit. */
int qko_reference_product(const float *x, const void *w, int type, int64_t K, int64_t N,
                          int64_t M, double *y, int threads)
{
    const int status = check_shape(type, K, N, M);
    if (status != 0 || M == 0)
        return status;
    const size_t row_bytes = (size_t)(K / QKO_QK) * (size_t)type_bytes(type);
    float *quantized = (float *)malloc((size_t)(M * K) * sizeof(float));
    if (!quantized)
        return 1;
    qko_q8_roundtrip(x, quantized, M * K);
    const uint8_t *base = (const uint8_t *)w;
#ifdef _OPENMP
    const int nt = threads > 0 ? threads : omp_get_num_procs();
#pragma omp parallel num_threads(nt)
#endif
    {
        float *decoded = (float *)malloc((size_t)K * sizeof(float));
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
        for (int64_t n = 0; n < N; ++n) {
            dequantize_row(type, base + (size_t)n * row_bytes, decoded, K);
            for (int64_t m = 0; m < M; ++m) {
                const float *q = quantized + m * K;
                double acc = 0.0;
                for (int64_t k = 0; k < K; ++k)
                    acc += (double)q[k] * (double)decoded[k];
                y[m * N + n] = acc;
            }
        }
        free(decoded);
    }
    (void)threads;
    free(quantized);
    return 0;
}

int qko_reference_product_f32(const float *x, const void *w, int type, int64_t K,
                              int64_t N, int64_t M, float *y, int threads)
{
    const int status = check_shape(type, K, N, M);
    if (status != 0 || M == 0)
        return status;
    const size_t row_bytes = (size_t)(K / QKO_QK) * (size_t)type_bytes(type);
    float *quantized = (float *)malloc((size_t)(M * K) * sizeof(float));
    if (!quantized)
        return 1;
    qko_q8_roundtrip(x, quantized, M * K);
    const uint8_t *base = (const uint8_t *)w;
#ifdef _OPENMP
    const int nt = threads > 0 ? threads : omp_get_num_procs();
#pragma omp parallel num_threads(nt)
#endif
    {
        float *decoded = (float *)malloc((size_t)K * sizeof(float));
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
        for (int64_t n = 0; n < N; ++n) {
            dequantize_row(type, base + (size_t)n * row_bytes, decoded, K);
            for (int64_t m = 0; m < M; ++m) {
                const float *q = quantized + m * K;
                float acc = 0.0f;
                for (int64_t k = 0; k < K; ++k)
                    acc += q[k] * decoded[k];
                y[m * N + n] = acc;
            }
        }
        free(decoded);
    }
    (void)threads;
    free(quantized);
    return 0;
}

static int dp4a(uint32_t a, const int8_t *x)
{
    int acc = 0;
    for (int i = 0; i < 4; ++i)
        acc += (int)(int8_t)(uint8_t)(a >> (8 * i)) * (int)x[i];
    return acc;
}

static uint32_t load_u32(const uint8_t *p)
{
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

/* src/cuda/matmul.cu:24-54 for one lane (group = lane/4, 8 weights at (lane%4)*8). */
static float lane_dot_q4k(const uint8_t *block, const int8_t *codes, const float *scales,
                          int lane)
{
    const int group = lane / 4;
    const int offset = (lane % 4) * 8;
    const int8_t *x = codes + group * 32 + offset;
    const uint8_t *packed = block + 16 + (group / 2) * 32 + offset;
    const int shift = (group % 2) * 4;
    const uint32_t a = (load_u32(packed) >> shift) & 0x0f0f0f0fu;
    const uint32_t b = (load_u32(packed + 4) >> shift) & 0x0f0f0f0fu;
    const int dot = dp4a(a, x) + dp4a(b, x + 4);
    int input_sum = 0;
    for (int i = 0; i < 8; ++i)
        input_sum += x[i];
    int scale, minimum;
    qko_get_scale_min_k4(group, block + 4, &scale, &minimum);
    const float d = load_fp16(block);
    const float dmin = load_fp16(block + 2);
    const float first = d * (float)scale * (float)dot;
    const float second = dmin * (float)minimum * (float)input_sum;
    return scales[group] * (first - second);
}

/* src/cuda/matmul.cu:61-84 for one lane. */
static float lane_dot_q6k(const uint8_t *block, const int8_t *codes, const float *scales,
                          int lane)
{
    const int group = lane / 4;
    const int offset = (lane % 4) * 8;
    const int8_t *x = codes + group * 32 + offset;
    const int half = group / 4, plane = group % 4;
    int dot = 0;
    for (int word = 0; word < 2; ++word) {
        const uint32_t low = load_u32(block + half * 64 + (plane % 2) * 32 + offset + word * 4);
        const uint32_t high = load_u32(block + 128 + half * 32 + offset + word * 4);
        const uint32_t codes4 = ((low >> (4 * (plane / 2))) & 0x0f0f0f0fu) |
                                (((high >> (2 * plane)) & 0x03030303u) << 4);
        for (int i = 0; i < 4; ++i)
            dot += ((int)((codes4 >> (8 * i)) & 0xFFu) - 32) * (int)x[word * 4 + i];
    }
    const int scale = ((const int8_t *)(block + 192))[group * 2 + offset / 16];
    const float d = load_fp16(block + 208);
    return scales[group] * (d * (float)scale * (float)dot);
}

int qko_integer_product(const float *x, const void *w, int type, int64_t K, int64_t N,
                        int64_t M, float *y)
{
    const int status = check_shape(type, K, N, M);
    if (status != 0 || M == 0)
        return status;
    const int64_t blocks = K / QKO_QK;
    const size_t bytes = (size_t)type_bytes(type);
    int8_t *codes = (int8_t *)malloc((size_t)(M * K));
    float *scales = (float *)malloc((size_t)(M * K / 32) * sizeof(float));
    if (!codes || !scales) {
        free(codes);
        free(scales);
        return 1;
    }
    qko_quantize_q8(x, codes, scales, M * K);
    const uint8_t *base = (const uint8_t *)w;
    for (int64_t m = 0; m < M; ++m) {
        for (int64_t n = 0; n < N; ++n) {
            float sum = 0.0f;
            for (int64_t b = 0; b < blocks; ++b) {
                const uint8_t *block = base + ((size_t)n * (size_t)blocks + (size_t)b) * bytes;
                const int8_t *cx = codes + m * K + b * QKO_QK;
                const float *sx = scales + m * (K / 32) + b * 8;
                for (int lane = 0; lane < 32; ++lane)
                    sum += type == QKO_TYPE_Q4_K ? lane_dot_q4k(block, cx, sx, lane)
                                                 : lane_dot_q6k(block, cx, sx, lane);
            }
            y[m * N + n] = sum;
        }
    }
    free(codes);
    free(scales);
    return 0;
}

/* ---------------------------------------------------------- neighbours --- */

/* src/cuda/silu_multiply.cu:6-12 (host libm expf, not a device expf). */
void qko_silu_multiply(const float *gate, const float *up, float *out, int64_t count)
{
    for (int64_t i = 0; i < count; ++i) {
        const float v = gate[i];
        out[i] = (v / (1.0f + expf(-v))) * up[i];
    }
}

/* src/cuda/rms_norm.cu:6-24: out = x * rsqrt(mean(x^2) + eps) * scale per
 * row of `width` values, products left to right in float. The sum of squares
 * is accumulated in double (the reference's per-thread float sums and tree
 * reduction, and its approximate rsqrtf, are not restated: they move the
 * result by a few ulp) and 1/sqrt is taken in double, then rounded. */
void qko_rms_norm(const float *x, const float *scale, float *out, int64_t rows, int64_t width,
                  float eps)
{
    for (int64_t r = 0; r < rows; ++r) {
        const float *xr = x + r * width;
        double sum = 0.0;
        for (int64_t i = 0; i < width; ++i) sum += (double)xr[i] * (double)xr[i];
        const float inv = (float)(1.0 / sqrt((double)(float)(sum / (double)width) + (double)eps));
        for (int64_t i = 0; i < width; ++i) out[r * width + i] = (xr[i] * inv) * scale[i];
    }
}

/* src/cuda/argmax.cu:25-98: the candidate starts at (SIZE_MAX, -inf) (:13-15)
 * and is replaced only by a strictly greater score (:32), ties across threads
 * going to the lower index (:19-23): the first index of the largest value;
 * NaN and -inf never win; if nothing wins, SIZE_MAX, which the uint32_t
 * return (:96) makes 0xFFFFFFFF. */
int64_t qko_argmax(const float *v, int64_t count)
{
    int64_t best = -1;
    float score = -INFINITY;
    for (int64_t i = 0; i < count; ++i)
        if (v[i] > score) {
            score = v[i];
            best = i;
        }
    return best < 0 ? (int64_t)0xFFFFFFFFu : best;
}

/* ------------------------------------------------------------ synthetic --- */

uint64_t qko_mix64(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

uint64_t qko_word(uint64_t seed, uint64_t i)
{
    return qko_mix64(seed + (i + 1) * 0x9E3779B97F4A7C15ull);
}

static float u24(uint64_t w)
{
    return (float)(w >> 40) * (1.0f / 16777216.0f);
}

static void put_u64(uint8_t *p, uint64_t w)
{
    for (int i = 0; i < 8; ++i)
        p[i] = (uint8_t)(w >> (8 * i));
}

void qko_synth_superblocks(void *w, int type, int64_t N, int64_t K, uint64_t seed,
                           float dmax, float dminmax)
{
    const int64_t blocks = N * (K / QKO_QK);
    uint8_t *out = (uint8_t *)w;
    if (type == QKO_TYPE_Q4_K) {
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
        for (int64_t b = 0; b < blocks; ++b) {
            uint8_t *block = out + b * QKO_Q4K_BYTES;
            const uint64_t base = (uint64_t)b * 20u;
            const uint16_t d = qko_fp32_to_fp16(u24(qko_word(seed, base + 0)) * dmax);
            const uint16_t dmin = qko_fp32_to_fp16(u24(qko_word(seed, base + 1)) * dminmax);
            block[0] = (uint8_t)d;
            block[1] = (uint8_t)(d >> 8);
            block[2] = (uint8_t)dmin;
            block[3] = (uint8_t)(dmin >> 8);
            uint8_t sc[16];
            put_u64(sc, qko_word(seed, base + 2));
            put_u64(sc + 8, qko_word(seed, base + 3));
            memcpy(block + 4, sc, 12);
            for (int i = 0; i < 16; ++i)
                put_u64(block + 16 + 8 * i, qko_word(seed, base + 4 + (uint64_t)i));
        }
    } else {
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
        for (int64_t b = 0; b < blocks; ++b) {
            uint8_t *block = out + b * QKO_Q6K_BYTES;
            const uint64_t base = (uint64_t)b * 27u;
            for (int i = 0; i < 24; ++i) /* ql[128] then qh[64] */
                put_u64(block + 8 * i, qko_word(seed, base + (uint64_t)i));
            uint8_t raw[16];
            put_u64(raw, qko_word(seed, base + 24));
            put_u64(raw + 8, qko_word(seed, base + 25));
            for (int i = 0; i < 16; ++i)
                block[192 + i] = (uint8_t)(int8_t)((int)(raw[i] & 127) - 64);
            const uint16_t d = qko_fp32_to_fp16(u24(qko_word(seed, base + 26)) * dmax);
            block[208] = (uint8_t)d;
            block[209] = (uint8_t)(d >> 8);
        }
    }
}

void qko_synth_normal(float *x, int64_t count, uint64_t seed)
{
    const double two_pi = 6.283185307179586476925286766559;
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
    for (int64_t i = 0; i < count; ++i) {
        const double u1 = 1.0 - (double)u24(qko_word(seed, 2 * (uint64_t)i));
        const double u2 = (double)u24(qko_word(seed, 2 * (uint64_t)i + 1));
        x[i] = (float)(sqrt(-2.0 * log(u1)) * cos(two_pi * u2));
    }
}
