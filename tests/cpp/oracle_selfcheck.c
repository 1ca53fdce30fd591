/* Runs every oracle function on small seeded inputs and checks properties the
 * mathematics fixes, so that a host sanitizer build (ASan/UBSan) exercises all
 * of oracle/qk_oracle.c: the dequantised product equals the reference product
 * computed from the dequantised rows, the integer decomposition agrees with it,
 * Q8 round trip = codes x scale, argmax finds a planted maximum. Exit status 0
 * when every check holds. */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "qk_oracle.h"

static int failures = 0;
#define CHECK(cond)                                                   \
    do {                                                              \
        if (!(cond)) {                                                \
            fprintf(stderr, "check failed: %s (line %d)\n", #cond, __LINE__); \
            ++failures;                                               \
        }                                                             \
    } while (0)

int main(void) {
    enum { K = 512, N = 7, M = 3 };
    float x[M * K], q[M * K], deq[N * K];
    int8_t codes[M * K];
    float scales[M * K / 32];
    double y[M * N];
    float yf[M * N], yi[M * N];
    qko_synth_normal(x, M * K, 11);
    for (int t = 0; t < 2; ++t) {
        const int type = t ? QKO_TYPE_Q6_K : QKO_TYPE_Q4_K;
        const size_t rb = (size_t)(K / 256) * (t ? QKO_Q6K_BYTES : QKO_Q4K_BYTES);
        unsigned char *w = malloc(rb * N);
        qko_synth_superblocks(w, type, N, K, 99 + t, 0.01f, 0.01f);
        CHECK(qko_dequantize_rows(w, deq, N, K, rb, type) == 0);
        CHECK(qko_reference_product(x, w, type, K, N, M, y, 1) == 0);
        CHECK(qko_reference_product_f32(x, w, type, K, N, M, yf, 2) == 0);
        CHECK(qko_integer_product(x, w, type, K, N, M, yi) == 0);
        qko_q8_roundtrip(x, q, M * K);
        for (int m = 0; m < M; ++m)
            for (int n = 0; n < N; ++n) {
                double e = 0.0;
                for (int k = 0; k < K; ++k) e += (double)q[m * K + k] * (double)deq[n * K + k];
                CHECK(e == y[m * N + n]);
                CHECK(fabs(yf[m * N + n] - e) <= 1e-4 * (1.0 + fabs(e)));
                CHECK(fabs(yi[m * N + n] - e) <= 1e-4 * (1.0 + fabs(e)));
            }
        CHECK(qko_dequantize_rows(w, deq, N, K, rb, 13) == 2);
        free(w);
    }
    qko_quantize_q8(x, codes, scales, M * K);
    for (int i = 0; i < M * K; ++i) CHECK(q[i] == (float)codes[i] * scales[i / 32]);
    float g[64], u[64], o[64], sc[K], nx[K];
    for (int i = 0; i < 64; ++i) {
        g[i] = (float)i - 32.0f;
        u[i] = 0.5f;
    }
    qko_silu_multiply(g, u, o, 64);
    CHECK(o[32] == 0.0f && o[63] > 15.0f);
    for (int i = 0; i < K; ++i) sc[i] = 1.0f;
    qko_rms_norm(x, sc, nx, 1, K, 1e-6f);
    double ss = 0.0;
    for (int i = 0; i < K; ++i) ss += (double)nx[i] * nx[i];
    CHECK(fabs(ss / K - 1.0) < 1e-4);
    float v[100];
    for (int i = 0; i < 100; ++i) v[i] = (float)(i % 7);
    v[57] = 9.0f;
    CHECK(qko_argmax(v, 100) == 57);
    CHECK(qko_fp16_to_fp32(qko_fp32_to_fp16(0.5f)) == 0.5f);
    int s6, m6;
    const unsigned char field[12] = {1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12};
    qko_get_scale_min_k4(5, field, &s6, &m6);
    CHECK(s6 >= 0 && s6 < 64 && m6 >= 0 && m6 < 64);
    if (failures == 0) printf("oracle self-check: all checks passed\n");
    return failures ? 1 : 0;
}
