// Generic quantized linear: any shape, alignment, format and dtype.
//
// The fallback behind rq_qmatmul for requests the tuned kernels do not
// serve (K not a multiple of 16/64, unaligned pointers, very large K, f32
// activations with many rows).  One block per output feature n; its 256
// threads stride over k, the block reduces through LDS, once per token row.
// Same arithmetic as the tuned kernels: rowwise sums q*x and scales once,
// affine dequantizes each weight to f32 (u*s + b, rounded) before the product.
#include "common.hpp"

namespace rq {
namespace {

constexpr int TH = 256;

template <typename T> __device__ __forceinline__ float ld(const void *p, size_t i) {
    return (float)reinterpret_cast<const T *>(p)[i];
}

__global__ __launch_bounds__(TH) void k_qlinear_generic(const uint8_t *__restrict__ codes,
                                                        const float *__restrict__ scales,
                                                        const float *__restrict__ biases, int fmt, int64_t group,
                                                        const void *__restrict__ X, int x_f16, void *__restrict__ Y,
                                                        int y_f16, int64_t M, int64_t N, int64_t K) {
    __shared__ float red[TH / 64];
    const int64_t n = blockIdx.x;
    const int t = threadIdx.x;
    const uint8_t *wrow = codes + n * K;
    for (int64_t m = 0; m < M; ++m) {
        float acc = 0.0f;
        for (int64_t k = t; k < K; k += TH) {
            const float x = x_f16 ? ld<_Float16>(X, m * K + k) : ld<float>(X, m * K + k);
            float w;
            if (fmt == RQ_Q_ROWWISE_I8) {
                w = (float)(int8_t)wrow[k];
            } else {
#pragma clang fp contract(off)
                const int64_t g = (n * K + k) / group;
                const float p = (float)wrow[k] * scales[g];
                w = p + (biases ? biases[g] : 0.0f);
            }
            acc = __builtin_fmaf(w, x, acc);
        }
        for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 64);
        if (t % 64 == 0) red[t / 64] = acc;
        __syncthreads();
        if (t == 0) {
            float v = 0.0f;
            for (int i = 0; i < TH / 64; ++i) v += red[i];
            if (fmt == RQ_Q_ROWWISE_I8) v *= scales[n];
            if (y_f16) reinterpret_cast<_Float16 *>(Y)[m * N + n] = (_Float16)v;
            else reinterpret_cast<float *>(Y)[m * N + n] = v;
        }
        __syncthreads();
    }
}

}  // namespace

int launch_qlinear_generic(const rq_qweight &w, const void *x, rq_dtype xt, void *y, rq_dtype yt, int64_t m,
                           hipStream_t s) {
    if (w.n_out > 0x7fffffff) return fail(RQ_ERR_SHAPE, "n_out too large for the generic kernel");
    hipLaunchKernelGGL(k_qlinear_generic, dim3((unsigned)w.n_out), dim3(TH), 0, s, (const uint8_t *)w.codes,
                       w.scales, w.biases, (int)w.format, (int64_t)(w.group > 0 ? w.group : 1), x,
                       xt == RQ_F16 ? 1 : 0, y, yt == RQ_F16 ? 1 : 0, m, w.n_out, w.k_in);
    RQ_LAUNCH_CHECK();
    return RQ_OK;
}

}  // namespace rq
