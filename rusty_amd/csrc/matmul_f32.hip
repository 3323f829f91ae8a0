// f32 matmul family: the reference's per-token GEMMs on an f32 weight.
//
//   MM_AB  <- rusty-backend/src/kernels.wgsl:7-54    (`matmul_tiled`, C = A.B)
//   MM_ABT <- rusty-backend/src/kernels.wgsl:234-242 (`matmul_bt`,    C = A.B^T)
//   MM_ATB <- rusty-backend/src/kernels.wgsl:244-252 (`matmul_at`,    C = A^T.B)
//
// Every output is one f32 accumulator updated in ascending k with a fused
// multiply-add, the order all three WGSL kernels use, so results are
// bit-identical to a sequential k-ascending fma loop regardless of tiling.
// Tiles are 64x64 per 256-thread block with 4x4 outputs per thread (16x the
// reuse of the reference's 16x16 one-output-per-invocation tiles); operands
// are staged through LDS k-major so the inner loop reads broadcast rows.
// Out-of-range rows/columns/k load as zero, which leaves every in-range
// accumulator unchanged.
#include "common.hpp"

namespace rq {
namespace {

constexpr int BM = 64, BN = 64, BK = 16, TH = 256;

template <int V>
__device__ __forceinline__ float load_a(const float *a, int64_t r, int64_t c, int64_t m, int64_t k) {
    // logical A[r, c] with r < m, c < k
    if (r >= m || c >= k) return 0.0f;
    if constexpr (V == MM_ATB) return a[c * m + r];  // A stored [k, m]
    else return a[r * k + c];
}

template <int V>
__device__ __forceinline__ float load_b(const float *b, int64_t r, int64_t c, int64_t k, int64_t n) {
    // logical B[r, c] with r < k, c < n
    if (r >= k || c >= n) return 0.0f;
    if constexpr (V == MM_ABT) return b[c * k + r];  // B stored [n, k]
    else return b[r * n + c];
}

template <int V>
__global__ __launch_bounds__(TH) void k_matmul_f32(const float *__restrict__ a, const float *__restrict__ b,
                                                   float *__restrict__ out, int64_t m, int64_t k, int64_t n) {
    __shared__ float As[BK][BM + 1];
    __shared__ float Bs[BK][BN + 1];
    const int t = threadIdx.x;
    const int tx = t % 16, ty = t / 16;
    const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * BN;

    float acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = 0.0f;

    for (int64_t k0 = 0; k0 < k; k0 += BK) {
        // A tile: BM x BK.  Coalesce along the contiguous dimension.
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if constexpr (V == MM_ATB) {
                const int r = t % 64, c = t / 64 + 4 * i;
                As[c][r] = load_a<V>(a, m0 + r, k0 + c, m, k);
            } else {
                const int c = t % 16, r = t / 16 + 16 * i;
                As[c][r] = load_a<V>(a, m0 + r, k0 + c, m, k);
            }
        }
        // B tile: BK x BN.
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if constexpr (V == MM_ABT) {
                const int c = t % 16, r = t / 16 + 16 * i;
                Bs[c][r] = load_b<V>(b, k0 + c, n0 + r, k, n);
            } else {
                const int r = t % 64, c = t / 64 + 4 * i;
                Bs[c][r] = load_b<V>(b, k0 + c, n0 + r, k, n);
            }
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < BK; ++kk) {
            float av[4], bv[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) av[i] = As[kk][ty + 16 * i];
#pragma unroll
            for (int j = 0; j < 4; ++j) bv[j] = Bs[kk][tx + 16 * j];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_fmaf(av[i], bv[j], acc[i][j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t r = m0 + ty + 16 * i, c = n0 + tx + 16 * j;
            if (r < m && c < n) out[r * n + c] = acc[i][j];
        }
}

}  // namespace

int launch_matmul_f32(int variant, const float *a, const float *b, float *out, int64_t m, int64_t k, int64_t n,
                      hipStream_t s) {
    if (m == 0 || n == 0) return RQ_OK;
    const int64_t gx = cdiv(n, BN), gy = cdiv(m, BM);
    if (gx > 0x7fffffff || gy > 65535)
        return fail(RQ_ERR_SHAPE, "matmul grid too large (m=%lld n=%lld)", (long long)m, (long long)n);
    const dim3 grid((unsigned)gx, (unsigned)gy), block(TH);
    // k == 0 runs the same kernel: the k loop is empty and zeros are stored.
    switch (variant) {
    case MM_AB: hipLaunchKernelGGL(k_matmul_f32<MM_AB>, grid, block, 0, s, a, b, out, m, k, n); break;
    case MM_ABT: hipLaunchKernelGGL(k_matmul_f32<MM_ABT>, grid, block, 0, s, a, b, out, m, k, n); break;
    case MM_ATB: hipLaunchKernelGGL(k_matmul_f32<MM_ATB>, grid, block, 0, s, a, b, out, m, k, n); break;
    default: return fail(RQ_ERR_INVALID_ARGUMENT, "unknown matmul variant %d", variant);
    }
    RQ_LAUNCH_CHECK();
    return RQ_OK;
}

}  // namespace rq
