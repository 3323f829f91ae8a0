/*
 * oracle.c -- CPU restatement of Rusty's quantized-linear hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker that the HIP product
 * path is compared against.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it; the product library never links
 * or calls it.
 *
 * Every function cites the reference file:line whose behaviour it restates
 * (paths relative to the reference repository root).  The reference itself is
 * Rust + WGSL on wgpu and cannot be built here (no cargo/rustc, no Vulkan ICD),
 * so there is no oracle/_ref build; how each function is pinned without it is
 * listed below and exercised in tests/test_oracle.py.
 *
 *   orc_dequantize          rusty-backend/src/kernels.wgsl:153-166   pinned: known answer from
 *                           rusty-loader/examples/load_and_run.rs:18-34, byte-order / tail cases
 *   orc_affine_dequantize   rusty-backend/src/kernels.wgsl:379-400   pinned: closed forms
 *                           (s=1,b=0 -> exact bytes; power-of-two scales; group boundaries;
 *                           independent f64 emulation of the two roundings)
 *   orc_rowwise_dequantize  BASELINE per-row int8 convention f32(q)*s  pinned: closed forms
 *   orc_matmul              rusty-backend/src/kernels.wgsl:7-54      pinned: integer-valued brute
 *                           force vs numpy f64, identity known answer (examples/ops_test.rs:13-17)
 *   orc_matmul_bt           rusty-backend/src/kernels.wgsl:234-242   pinned: as orc_matmul
 *   orc_matmul_at           rusty-backend/src/kernels.wgsl:244-252   pinned: as orc_matmul
 *   orc_qlinear_truth       f64 truth of Y = X . deq(W)^T            pinned: numpy f64 einsum on
 *                           small shapes, integer-exact cases
 *   orc_ref_linear          the reference's Linear path: load-time dequantize to f32
 *                           (orc_ref_dequantize_linear), then per forward the matmul_tiled
 *                           k-ascending f32 sum on the [in,out] Linear weight (orc_ref_forward,
 *                           rusty-graph/src/lib.rs:69-70).  OpenMP; orc_ref_forward is the CPU
 *                           baseline that bench.py times.  pinned: equals orc_matmul on the
 *                           oracle-dequantized weight.
 *   orc_swiglu_truth        rusty-graph/src/lib.rs:317-323 (silu(gate) * up, then down) in f64
 *
 * Compile with -ffp-contract=off: the unfused variants must round after the
 * multiply and again after the add, exactly as written in the WGSL.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>
#include <stdlib.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* byte j of the little-endian u32 word stream (kernels.wgsl:159-165, :392-393) */
static inline uint32_t byte_at(const uint32_t *words, size_t i) {
    return (words[i >> 2] >> (8u * (uint32_t)(i & 3u))) & 0xFFu;
}

/* kernels.wgsl:153-166 (`dequantize`), host lib.rs:4872-4899.
 * out[4i+j] = f32((word_i >> 8j) & 0xFF) for every word i < n_words and
 * 4i+j < n_out.  The WGSL guards each of the four writes on arrayLength(out);
 * the host grid derives from the input's element count.  Here every word is
 * covered (the intended semantics). */
void orc_dequantize(const uint32_t *words, size_t n_words, float *out, size_t n_out) {
    size_t n = n_words * 4u;
    if (n > n_out) n = n_out;
    for (size_t i = 0; i < n; ++i) out[i] = (float)byte_at(words, i);
}

/* kernels.wgsl:379-400 (`affine_dequantize`), host lib.rs:4939-4990.
 * out[i] = f32(u8_i) * scales[i/group] + biases[i/group], group = 64 in the
 * reference (kernels.wgsl:395).  fused = 0: the multiply and the add each
 * round to f32 (as written); fused = 1: one fmaf (what a backend compiler that
 * contracts a*b+c produces).  Full coverage of [0, n): the reference's 2-D
 * dispatch fallback (lib.rs:4976-4987) leaves elements >= 65535*64 unwritten,
 * which is a defect this restatement does not reproduce. */
void orc_affine_dequantize(const uint32_t *words, const float *scales, const float *biases,
                           float *out, size_t n, uint32_t group, int fused) {
    for (size_t i = 0; i < n; ++i) {
        float u = (float)byte_at(words, i);
        size_t g = i / group;
        if (fused) {
            out[i] = fmaf(u, scales[g], biases[g]);
        } else {
            volatile float p = u * scales[g];
            out[i] = p + biases[g];
        }
    }
}

/* Per-output-row signed int8 convention of the benchmark configs:
 * W[n,k] = f32(q[n,k]) * scale[n].  One rounding (q*s is exact in f64 and
 * rounded once to f32), so contraction cannot change it. */
void orc_rowwise_dequantize(const int8_t *q, const float *scales, float *out, size_t N, size_t K) {
    for (size_t n = 0; n < N; ++n)
        for (size_t k = 0; k < K; ++k) out[n * K + k] = (float)q[n * K + k] * scales[n];
}

/* f32 accumulation step `acc = acc + a*b` (kernels.wgsl:46, :240, :250). */
static inline float acc_step(float acc, float a, float b, int fused) {
    if (fused) return fmaf(a, b, acc);
    volatile float p = a * b;
    return acc + p;
}

/* kernels.wgsl:7-54 (`matmul_tiled`), host lib.rs:4403-4453.
 * C[r,c] = sum_{k ascending} A[r,k]*B[k,c]; A [M,K], B [K,N], C [M,N] row-major.
 * The 16-wide LDS tiles zero-pad and then add k in ascending order, so the
 * f32 sequence is exactly the k-ascending one (padding adds +0*0 terms, which
 * leave a finite accumulator unchanged). */
void orc_matmul(const float *A, const float *B, float *C, int M, int K, int N, int fused) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < M; ++r)
        for (int c = 0; c < N; ++c) {
            float acc = 0.0f;
            for (int k = 0; k < K; ++k) acc = acc_step(acc, A[(size_t)r * K + k], B[(size_t)k * N + c], fused);
            C[(size_t)r * N + c] = acc;
        }
}

/* kernels.wgsl:234-242 (`matmul_bt`), host lib.rs:4299-4349: C = A . B^T,
 * A [M,K], B [N,K]. */
void orc_matmul_bt(const float *A, const float *B, float *C, int M, int K, int N, int fused) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < M; ++r)
        for (int c = 0; c < N; ++c) {
            float acc = 0.0f;
            for (int k = 0; k < K; ++k) acc = acc_step(acc, A[(size_t)r * K + k], B[(size_t)c * K + k], fused);
            C[(size_t)r * N + c] = acc;
        }
}

/* kernels.wgsl:244-252 (`matmul_at`), host lib.rs:4351-4401: C = A^T . B with
 * A [K,M] (the host reads m = a.shape[1], k = a.shape[0]), B [K,N]. */
void orc_matmul_at(const float *A, const float *B, float *C, int M, int K, int N, int fused) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < M; ++r)
        for (int c = 0; c < N; ++c) {
            float acc = 0.0f;
            for (int k = 0; k < K; ++k) acc = acc_step(acc, A[(size_t)k * M + r], B[(size_t)k * N + c], fused);
            C[(size_t)r * N + c] = acc;
        }
}

/* Dequantized weight element in f64 (exact: u*s and q*s are exact in f64;
 * the affine add is done in f64 too, so this is the mathematical value of the
 * quantized weight, not a rounded one). mode 0: signed per-row; mode 1: the
 * reference's unsigned affine group format (kernels.wgsl:392-399). */
static inline double wq_f64(const void *codes, const float *scales, const float *biases, int mode,
                            size_t group, size_t n, size_t k, size_t K) {
    size_t i = n * K + k;
    if (mode == 0) return (double)((const int8_t *)codes)[i] * (double)scales[n];
    size_t g = i / group;
    double u = (double)((const uint8_t *)codes)[i];
    return u * (double)scales[g] + (biases ? (double)biases[g] : 0.0);
}

/* f64 truth of Y[m,n] = sum_k X[m,k] * deq(W)[n,k]  (W is [out,in], i.e. the
 * `matmul_bt` orientation, kernels.wgsl:234-242).  X is given as f32 values
 * (already rounded to f16 by the caller when the device input is f16). */
void orc_qlinear_truth(const void *codes, const float *scales, const float *biases, int mode,
                       int group, const float *X, double *Y, int M, int N, int K) {
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; ++n)
        for (int m = 0; m < M; ++m) {
            double acc = 0.0;
            for (int k = 0; k < K; ++k)
                acc += (double)X[(size_t)m * K + k] * wq_f64(codes, scales, biases, mode, (size_t)group, n, k, K);
            Y[(size_t)m * N + n] = acc;
        }
}

/* The reference's Linear path, restated in its two steps:
 *   1. load time: dequantize the weight to f32 ([out,in], one rounding per
 *      element for the per-row mode, mul-then-add for the affine mode:
 *      kernels.wgsl:379-400, called from rusty-loader/src/lib.rs:209);
 *   2. every forward: Y = X . W with W the Linear weight [in,out]
 *      (rusty-graph/src/lib.rs:69-70) and matmul_tiled's k-ascending f32 sum
 *      (kernels.wgsl:7-54), each step contracted to one fma (what Metal/Vulkan
 *      shader compilers emit for `acc = acc + a*b`; orc_matmul offers both).
 * wbuf holds the f32 weight as [out,in] (wbuf[n*K+k] == W_linear[k][n]) so one
 * output's k run is contiguous.  OpenMP over output features; each returns
 * the thread count used. */
int orc_ref_dequantize_linear(const void *codes, const float *scales, const float *biases, int mode, int group,
                              float *wbuf, int N, int K) {
    int threads = 1;
#pragma omp parallel
    {
#ifdef _OPENMP
#pragma omp single
        threads = omp_get_num_threads();
#endif
#pragma omp for schedule(static)
        for (int n = 0; n < N; ++n)
            for (int k = 0; k < K; ++k) {
                size_t i = (size_t)n * K + k;
                float w;
                if (mode == 0) {
                    w = (float)((const int8_t *)codes)[i] * scales[n];
                } else {
                    size_t g = i / (size_t)group;
                    volatile float p = (float)((const uint8_t *)codes)[i] * scales[g];
                    w = p + (biases ? biases[g] : 0.0f);
                }
                wbuf[i] = w;
            }
    }
    return threads;
}

int orc_ref_forward(const float *wbuf, const float *X, float *Y, int M, int N, int K) {
    int threads = 1;
#pragma omp parallel
    {
#ifdef _OPENMP
#pragma omp single
        threads = omp_get_num_threads();
#endif
#pragma omp for schedule(static)
        for (int n = 0; n < N; ++n)
            for (int m = 0; m < M; ++m) {
                float acc = 0.0f;
                const float *w = wbuf + (size_t)n * K;
                const float *x = X + (size_t)m * K;
                for (int k = 0; k < K; ++k) acc = fmaf(x[k], w[k], acc);
                Y[(size_t)m * N + n] = acc;
            }
    }
    return threads;
}

int orc_ref_linear(const void *codes, const float *scales, const float *biases, int mode, int group,
                   const float *X, float *Y, float *wbuf, int M, int N, int K) {
    orc_ref_dequantize_linear(codes, scales, biases, mode, group, wbuf, N, K);
    return orc_ref_forward(wbuf, X, Y, M, N, K);
}

/* rusty-graph/src/lib.rs:317-323 (`MLP::forward`): down( silu(gate(x)) * up(x) ),
 * silu(v) = v / (1 + exp(-v)) (kernels.wgsl:104-113), in f64 from f64 truth
 * projections.  If h_round_f16 != 0 the intermediate h is rounded to f16 the
 * way a device pipeline that stores h in f16 does, which is what the GPU path
 * computes; hbuf is caller scratch of M*I doubles. */
static double round_f16(double v);
void orc_swiglu_truth(const int8_t *wg, const float *sg, const int8_t *wu, const float *su,
                      const int8_t *wd, const float *sd, const float *X, double *Y, double *hbuf,
                      int M, int H, int I, int h_round_f16) {
#pragma omp parallel for schedule(static)
    for (int i = 0; i < I; ++i)
        for (int m = 0; m < M; ++m) {
            double g = 0.0, u = 0.0;
            for (int k = 0; k < H; ++k) {
                double x = (double)X[(size_t)m * H + k];
                g += x * (double)wg[(size_t)i * H + k] * (double)sg[i];
                u += x * (double)wu[(size_t)i * H + k] * (double)su[i];
            }
            double h = g / (1.0 + exp(-g)) * u;
            hbuf[(size_t)m * I + i] = h_round_f16 ? round_f16(h) : h;
        }
#pragma omp parallel for schedule(static)
    for (int n = 0; n < H; ++n)
        for (int m = 0; m < M; ++m) {
            double acc = 0.0;
            for (int i = 0; i < I; ++i)
                acc += hbuf[(size_t)m * I + i] * (double)wd[(size_t)n * I + i] * (double)sd[n];
            Y[(size_t)m * H + n] = acc;
        }
}

/* IEEE binary16 round-to-nearest-even of a double (finite range only; values
 * beyond 65504 saturate to +-inf as the conversion does). */
static double round_f16(double v) {
    if (v == 0.0 || isnan(v)) return v;
    double a = fabs(v);
    if (a >= 65520.0) return v > 0 ? INFINITY : -INFINITY;
    int e;
    frexp(a, &e);             /* a = f * 2^e, f in [0.5,1) */
    int ulp_exp = e - 11;     /* 11 significant bits */
    if (ulp_exp < -24) ulp_exp = -24; /* subnormal spacing 2^-24 */
    double q = ldexp(1.0, ulp_exp);
    double r = nearbyint(a / q) * q;  /* default rounding mode is nearest-even */
    return v < 0 ? -r : r;
}

double orc_round_f16(double v) { return round_f16(v); }
