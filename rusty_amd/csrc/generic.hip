// Generic quantized linear: any shape, alignment, format and dtype.
//
// The fallback behind rq_qmatmul for requests the tuned kernels do not
// serve (K not a multiple of 16/64, unaligned pointers, very large K, f32
// activations with many rows).  One block per output feature n; its 256
// threads stride over k, the block reduces through LDS, once per token row.
// Same arithmetic as the tuned kernels: rowwise sums q*x and scales once,
// affine dequantizes each weight to f32 (u*s + b, rounded) before the product.
#include <algorithm>

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

__device__ __forceinline__ float silu(float v) { return v / (1.0f + expf(-v)); }

__device__ __forceinline__ float deq(const uint8_t *codes, const float *scales, const float *biases, int fmt,
                                     int64_t group, int64_t n, int64_t k, int64_t K) {
    if (fmt == RQ_Q_ROWWISE_I8) return (float)(int8_t)codes[n * K + k];
    {
#pragma clang fp contract(off)
        const int64_t g = (n * K + k) / group;
        const float p = (float)codes[n * K + k] * scales[g];
        return p + (biases ? biases[g] : 0.0f);
    }
}

// SwiGLU gate/up pass for any shape, format and activation dtype: one block
// per intermediate feature i, h[m, i] = silu(x.gate[i]) * (x.up[i]) in fp16.
__global__ __launch_bounds__(TH) void k_swiglu_generic(rq_qweight gate, rq_qweight up, const void *__restrict__ X,
                                                       int x_f16, _Float16 *__restrict__ H, int64_t M) {
    __shared__ float red[2][TH / 64];
    const int64_t i = blockIdx.x, K = gate.k_in, I = gate.n_out;
    const int t = threadIdx.x;
    const int64_t gg = gate.group > 0 ? gate.group : 1, gu = up.group > 0 ? up.group : 1;
    for (int64_t m = 0; m < M; ++m) {
        float ag = 0.0f, au = 0.0f;
        for (int64_t k = t; k < K; k += TH) {
            const float x = x_f16 ? ld<_Float16>(X, m * K + k) : ld<float>(X, m * K + k);
            ag = __builtin_fmaf(deq((const uint8_t *)gate.codes, gate.scales, gate.biases, gate.format, gg, i, k, K), x, ag);
            au = __builtin_fmaf(deq((const uint8_t *)up.codes, up.scales, up.biases, up.format, gu, i, k, K), x, au);
        }
        for (int o = 32; o > 0; o >>= 1) {
            ag += __shfl_xor(ag, o, 64);
            au += __shfl_xor(au, o, 64);
        }
        if (t % 64 == 0) {
            red[0][t / 64] = ag;
            red[1][t / 64] = au;
        }
        __syncthreads();
        if (t == 0) {
            float g = 0.0f, u = 0.0f;
            for (int w = 0; w < TH / 64; ++w) {
                g += red[0][w];
                u += red[1][w];
            }
            if (gate.format == RQ_Q_ROWWISE_I8) g *= gate.scales[i];
            if (up.format == RQ_Q_ROWWISE_I8) u *= up.scales[i];
            H[m * I + i] = (_Float16)(silu(g) * u);
        }
        __syncthreads();
    }
}

// h = silu(g) * u elementwise on fp16 (the prefill SwiGLU epilogue).
__global__ __launch_bounds__(TH) void k_silu_mul(const _Float16 *__restrict__ G, const _Float16 *__restrict__ U,
                                                 _Float16 *__restrict__ H, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * TH + threadIdx.x; i < n; i += (int64_t)gridDim.x * TH)
        H[i] = (_Float16)(silu((float)G[i]) * (float)U[i]);
}

// The same, 8 values per thread per step (16-byte loads and stores).
__global__ __launch_bounds__(TH) void k_silu_mul8(const uint4 *__restrict__ G, const uint4 *__restrict__ U,
                                                  uint4 *__restrict__ H, int64_t n8) {
    typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
    for (int64_t i = (int64_t)blockIdx.x * TH + threadIdx.x; i < n8; i += (int64_t)gridDim.x * TH) {
        const half8_t g = __builtin_bit_cast(half8_t, G[i]), u = __builtin_bit_cast(half8_t, U[i]);
        half8_t h;
#pragma unroll
        for (int e = 0; e < 8; ++e) h[e] = (_Float16)(silu((float)g[e]) * (float)u[e]);
        H[i] = __builtin_bit_cast(uint4, h);
    }
}

}  // namespace

int launch_swiglu_generic(const rq_qweight &gate, const rq_qweight &up, const void *x, rq_dtype xt, void *h, int64_t m,
                          hipStream_t s) {
    if (gate.n_out > 0x7fffffff) return fail(RQ_ERR_SHAPE, "intermediate size too large for the generic kernel");
    hipLaunchKernelGGL(k_swiglu_generic, dim3((unsigned)gate.n_out), dim3(TH), 0, s, gate, up, x, xt == RQ_F16 ? 1 : 0,
                       (_Float16 *)h, m);
    RQ_LAUNCH_CHECK();
    return RQ_OK;
}

int launch_silu_mul(const void *g, const void *u, void *h, int64_t n, hipStream_t s) {
    if (n % 8 == 0 && aligned(g, 16) && aligned(u, 16) && aligned(h, 16)) {
        const int64_t blocks = std::min<int64_t>(cdiv(n / 8, TH), 16384);
        if (blocks < 1) return RQ_OK;
        hipLaunchKernelGGL(k_silu_mul8, dim3((unsigned)blocks), dim3(TH), 0, s, (const uint4 *)g, (const uint4 *)u,
                           (uint4 *)h, n / 8);
        RQ_LAUNCH_CHECK();
        return RQ_OK;
    }
    int64_t blocks = cdiv(n, TH);
    if (blocks > 65536) blocks = 65536;
    if (blocks < 1) return RQ_OK;
    hipLaunchKernelGGL(k_silu_mul, dim3((unsigned)blocks), dim3(TH), 0, s, (const _Float16 *)g, (const _Float16 *)u,
                       (_Float16 *)h, n);
    RQ_LAUNCH_CHECK();
    return RQ_OK;
}

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
