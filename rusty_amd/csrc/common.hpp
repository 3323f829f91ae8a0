// Shared helpers of the gfx950 kernels and the C-ABI layer.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>
#include <stddef.h>

#include "rusty_hip.h"

namespace rq {

// Records a message for rq_last_error() and returns `status`.
int fail(int status, const char *fmt, ...);

// Evaluates a HIP call; on failure records the HIP error and returns RQ_ERR_HIP.
#define RQ_HIP_TRY(expr)                                                              \
    do {                                                                              \
        hipError_t rq_e_ = (expr);                                                    \
        if (rq_e_ != hipSuccess)                                                      \
            return ::rq::fail(RQ_ERR_HIP, "%s: %s (%s:%d)", #expr, hipGetErrorString(rq_e_), \
                              __FILE__, __LINE__);                                    \
    } while (0)

// Launch check: kernel launches report configuration errors via hipGetLastError.
#define RQ_LAUNCH_CHECK() RQ_HIP_TRY(hipGetLastError())

inline bool aligned(const void *p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Launchers implemented in the kernel translation units.  Arguments are
// validated by the C-ABI layer before these are called.
int launch_dequantize(const uint32_t *in, size_t n_words, float *out, size_t n_out, hipStream_t s);
int launch_affine_dequantize(const uint32_t *w, const float *scales, const float *biases, float *out,
                             size_t n, uint32_t group, bool fma, hipStream_t s);
int launch_rowwise_dequantize(const int8_t *q, const float *scales, float *out, int64_t n_rows,
                              int64_t k, hipStream_t s);
int launch_matmul_f32(int variant, const float *a, const float *b, float *out, int64_t m, int64_t k,
                      int64_t n, hipStream_t s);
int launch_gemv_decode(const rq_qweight &w, const void *x, void *y, rq_dtype yt, int m, hipStream_t s);
int launch_gemv_mfma(const rq_qweight &w, const void *x, void *y, rq_dtype yt, int m, hipStream_t s);
int launch_gemv(const rq_qweight &w, const void *x, rq_dtype xt, void *y, rq_dtype yt, int m,
                int num_cus, hipStream_t s);
int launch_gemm(const rq_qweight &w, const void *x, rq_dtype xt, void *y, rq_dtype yt, int64_t m,
                int num_cus, hipStream_t s);
int launch_qlinear_generic(const rq_qweight &w, const void *x, rq_dtype xt, void *y, rq_dtype yt,
                           int64_t m, hipStream_t s);
int launch_swiglu_decode(const rq_qweight &gate, const rq_qweight &up, const void *x, void *h, int m, hipStream_t s);
int launch_swiglu_mfma(const rq_qweight &gate, const rq_qweight &up, const void *x, void *h, int m, hipStream_t s);
int launch_swiglu_generic(const rq_qweight &gate, const rq_qweight &up, const void *x, rq_dtype xt, void *h,
                          int64_t m, hipStream_t s);
int launch_silu_mul(const void *g, const void *u, void *h, int64_t n, hipStream_t s);

enum MatmulVariant { MM_AB = 0, MM_ABT = 1, MM_ATB = 2 };

}  // namespace rq
