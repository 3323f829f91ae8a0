/* Plain-C client of librusty_hip.so: what a reference-side FFI binding does.
 * Built with gcc against include/rusty_hip.h only (no HIP, no C++ headers).
 * Checks, on the device: rq_affine_dequantize bit-exact against a C loop of
 * the reference formula (kernels.wgsl:379-400, multiply then add in f32),
 * rq_qmatmul against a double-precision loop, and two error statuses.
 * Prints "abi_example: OK" and exits 0 on success. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "rusty_hip.h"

#define CHECK(call)                                                                                   \
    do {                                                                                              \
        int st_ = (call);                                                                             \
        if (st_ != RQ_OK) {                                                                           \
            fprintf(stderr, "%s failed: %s (%s)\n", #call, rq_status_string(st_), rq_last_error()); \
            return 1;                                                                                 \
        }                                                                                             \
    } while (0)

static uint32_t lcg(uint32_t *s) { return *s = *s * 1664525u + 1013904223u; }

int main(void) {
    rq_ctx *ctx = NULL;
    CHECK(rq_ctx_create(0, &ctx));

    /* affine dequant: 8 rows x 256 codes, group 64 */
    enum { N = 8, K = 256, G = 64, NG = N * K / G };
    uint8_t codes[N * K];
    float scales[NG], biases[NG], want[N * K], got[N * K];
    uint32_t seed = 12345;
    for (int i = 0; i < N * K; ++i) codes[i] = (uint8_t)(lcg(&seed) >> 24);
    for (int g = 0; g < NG; ++g) {
        scales[g] = 0.001f + (float)(lcg(&seed) >> 8) / 16777216.0f * 0.019f;
        biases[g] = -128.0f * scales[g];
    }
    for (int i = 0; i < N * K; ++i) {
        volatile float p = (float)codes[i] * scales[i / G]; /* rounded product, then the add */
        want[i] = p + biases[i / G];
    }
    void *d_codes, *d_s, *d_b, *d_out, *d_x, *d_y;
    CHECK(rq_alloc(ctx, sizeof codes, &d_codes));
    CHECK(rq_alloc(ctx, sizeof scales, &d_s));
    CHECK(rq_alloc(ctx, sizeof biases, &d_b));
    CHECK(rq_alloc(ctx, sizeof got, &d_out));
    CHECK(rq_memcpy_h2d(ctx, d_codes, codes, sizeof codes, NULL));
    CHECK(rq_memcpy_h2d(ctx, d_s, scales, sizeof scales, NULL));
    CHECK(rq_memcpy_h2d(ctx, d_b, biases, sizeof biases, NULL));
    CHECK(rq_affine_dequantize(ctx, (const uint32_t *)d_codes, N * K / 4, (const float *)d_s, (const float *)d_b, NG,
                               (float *)d_out, N * K, G, 0, NULL));
    CHECK(rq_memcpy_d2h(ctx, got, d_out, sizeof got, NULL));
    if (memcmp(got, want, sizeof got) != 0) {
        fprintf(stderr, "affine dequant differs from the reference formula\n");
        return 1;
    }

    /* fused quantized linear, f32 in/out, m = 3 */
    enum { M = 3 };
    float x[M * K], y[M * N];
    for (int i = 0; i < M * K; ++i) x[i] = (float)(lcg(&seed) >> 8) / 16777216.0f - 0.5f;
    CHECK(rq_alloc(ctx, sizeof x, &d_x));
    CHECK(rq_alloc(ctx, sizeof y, &d_y));
    CHECK(rq_memcpy_h2d(ctx, d_x, x, sizeof x, NULL));
    rq_qweight w = {d_codes, (const float *)d_s, (const float *)d_b, N, K, RQ_Q_AFFINE_U8, G};
    CHECK(rq_qmatmul(ctx, &w, d_x, RQ_F32, d_y, RQ_F32, M, NULL));
    CHECK(rq_memcpy_d2h(ctx, y, d_y, sizeof y, NULL));
    double worst = 0.0, scale = 0.0;
    for (int m = 0; m < M; ++m)
        for (int n = 0; n < N; ++n) {
            double t = 0.0;
            for (int k = 0; k < K; ++k)
                t += (double)x[m * K + k] * ((double)codes[n * K + k] * scales[(n * K + k) / G] + biases[(n * K + k) / G]);
            worst = fmax(worst, fabs(t - y[m * N + n]));
            scale = fmax(scale, fabs(t));
        }
    if (worst > 1e-5 * scale + 1e-6) {
        fprintf(stderr, "qmatmul max |d| %.3g vs max |y| %.3g\n", worst, scale);
        return 1;
    }

    /* errors are returned, not raised */
    if (rq_qmatmul(ctx, NULL, d_x, RQ_F32, d_y, RQ_F32, M, NULL) != RQ_ERR_INVALID_ARGUMENT) return 1;
    w.format = 7;
    if (rq_qmatmul(ctx, &w, d_x, RQ_F32, d_y, RQ_F32, M, NULL) != RQ_ERR_INVALID_ARGUMENT) return 1;

    CHECK(rq_free(ctx, d_codes));
    CHECK(rq_free(ctx, d_s));
    CHECK(rq_free(ctx, d_b));
    CHECK(rq_free(ctx, d_out));
    CHECK(rq_free(ctx, d_x));
    CHECK(rq_free(ctx, d_y));
    CHECK(rq_ctx_destroy(ctx));
    printf("abi_example: OK (qmatmul max |d| %.3g of %.3g)\n", worst, scale);
    return 0;
}
