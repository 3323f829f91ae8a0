// Input gradient through a frozen quantized Linear (LoRA fine-tuning):
//
//   dX[m, k_in] = dY[m, n_out] . deq(W)[n_out, k_in]
//
// the `grad_a = matmul_bt(grad, b)` step of MatMulNode::backward
// (rusty-autograd/src/lib.rs:152-158) with b the load-time-dequantized f32
// weight in [in, out] layout (rusty-graph/src/lib.rs:69-70): since
// b[i, o] = deq(W)[o, i], matmul_bt(grad, b) = dY . deq(W) in the stored
// [out, in] orientation, so W is read as it lies, with no transpose.  The
// weight gradient is not formed (the weight is frozen).
//
// Tiling: 64x64 output tiles per 256-thread block, 4x4 outputs per thread,
// one f32 accumulator per output updated by fma in ascending n_out (the f32
// matmul family's order).  The weight tile is dequantized while it is staged
// -- per-row codes f32(q) * s[row] (one rounding), affine codes
// (f32(u) * s[g]) + b[g] (two roundings, no contraction), exactly the values
// rq_qweight_dequantize writes -- so dX is bit-identical to the f32 matmul on
// the dequantized weight without that weight ever existing in memory.
// Memory: 1 B per weight element instead of 4.  Steps of 32 along n_out; the
// next step's dY and code pieces are loaded into registers (8 codes and 8 dY
// values per thread) before the current step's fmas run, so a block's loads
// overlap its arithmetic (a few blocks per CU at prompt-sized m cannot hide
// the latency by occupancy alone: 512 x 4096 x 4096 took 730 us with
// single-buffered 16-step tiles).
#include "common.hpp"

namespace rq {
namespace {

constexpr int BM = 64, BN = 64, BK = 32, TH = 256;

// The dequantized value of code c of weight row `row`, column `col`.
template <int FMT>
__device__ __forceinline__ float deq1(uint32_t c, const float *scales, const float *biases, int group, int64_t row,
                                      int64_t col, int64_t k_in) {
    if constexpr (FMT == RQ_Q_ROWWISE_I8) {
        return (float)(int8_t)c * scales[row];
    } else {
        const int64_t g = (row * k_in + col) / group;
        float v;
        {
#pragma clang fp contract(off)
            v = (float)c * scales[g];
            v = v + (biases ? biases[g] : 0.0f);
        }
        return v;
    }
}

template <int FMT, bool DYF16, bool DXF16>
__global__ __launch_bounds__(TH) void k_qmatmul_dx(const uint8_t *__restrict__ codes, const float *__restrict__ scales,
                                                   const float *__restrict__ biases, int group,
                                                   const void *__restrict__ dyv, void *__restrict__ dxv, int64_t m,
                                                   int64_t n_out, int64_t k_in) {
    __shared__ float As[BK][BM + 1];  // dY^T tile: [n_out step][row of dX]
    __shared__ float Bs[BK][BN + 4];  // deq(W) tile: [n_out step][column of dX]
    const int t = threadIdx.x;
    const int tx = t % 16, ty = t / 16;
    const int64_t m0 = (int64_t)blockIdx.y * BM, c0 = (int64_t)blockIdx.x * BN;
    // this thread's staging pieces: dY row ar, entries ac..ac+7 of the step
    // (contiguous along n_out); weight row br of the step, columns bc..bc+7
    const int ar = t / 4, ac = (t % 4) * 8;
    const int br = t / 8, bc = (t % 8) * 8;
    const bool vec_w = k_in % 8 == 0 && (reinterpret_cast<uintptr_t>(codes) % 8) == 0;

    float ya[8];
    uint32_t wc[8];
    auto load = [&](int64_t k0) {
        const int64_t gr = m0 + ar;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int64_t gc = k0 + ac + e;
            float v = 0.0f;
            if (gr < m && gc < n_out) {
                const int64_t o = gr * n_out + gc;
                v = DYF16 ? (float)static_cast<const _Float16 *>(dyv)[o] : static_cast<const float *>(dyv)[o];
            }
            ya[e] = v;
        }
        const int64_t row = k0 + br, col = c0 + bc;
        if (row < n_out && vec_w && col + 8 <= k_in) {
            const uint2 q = *reinterpret_cast<const uint2 *>(codes + row * k_in + col);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                wc[e] = (q.x >> (8 * e)) & 0xFFu;
                wc[4 + e] = (q.y >> (8 * e)) & 0xFFu;
            }
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) wc[e] = row < n_out && col + e < k_in ? codes[row * k_in + col + e] : 0u;
        }
    };
    auto stage = [&](int64_t k0) {
#pragma unroll
        for (int e = 0; e < 8; ++e) As[ac + e][ar] = ya[e];
        const int64_t row = k0 + br, col = c0 + bc;
#pragma unroll
        for (int e = 0; e < 8; ++e)
            Bs[br][bc + e] = row < n_out && col + e < k_in
                                 ? deq1<FMT>(wc[e], scales, biases, group, row, col + e, k_in)
                                 : 0.0f;
    };

    float acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = 0.0f;

    if (n_out > 0) load(0);
    for (int64_t k0 = 0; k0 < n_out; k0 += BK) {
        stage(k0);
        __syncthreads();
        if (k0 + BK < n_out) load(k0 + BK);  // in flight while this step's fmas run
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
            const int64_t r = m0 + ty + 16 * i, c = c0 + tx + 16 * j;
            if (r < m && c < k_in) {
                if constexpr (DXF16) static_cast<_Float16 *>(dxv)[r * k_in + c] = (_Float16)acc[i][j];
                else static_cast<float *>(dxv)[r * k_in + c] = acc[i][j];
            }
        }
}

template <int FMT, bool DYF16>
int launch_fmt(const rq_qweight &w, const void *dy, void *dx, bool dxf16, int64_t m, dim3 grid, hipStream_t s) {
    const uint8_t *codes = static_cast<const uint8_t *>(w.codes);
    if (dxf16)
        hipLaunchKernelGGL((k_qmatmul_dx<FMT, DYF16, true>), grid, dim3(TH), 0, s, codes, w.scales, w.biases, w.group,
                           dy, dx, m, w.n_out, w.k_in);
    else
        hipLaunchKernelGGL((k_qmatmul_dx<FMT, DYF16, false>), grid, dim3(TH), 0, s, codes, w.scales, w.biases,
                           w.group, dy, dx, m, w.n_out, w.k_in);
    RQ_LAUNCH_CHECK();
    return RQ_OK;
}

}  // namespace

int launch_qmatmul_dx(const rq_qweight &w, const void *dy, rq_dtype dyt, void *dx, rq_dtype dxt, int64_t m,
                      hipStream_t s) {
    const int64_t gx = cdiv(w.k_in, BN), gy = cdiv(m, BM);
    if (gx > 0x7fffffff || gy > 65535)
        return fail(RQ_ERR_SHAPE, "input-gradient grid too large (m=%lld k_in=%lld)", (long long)m,
                    (long long)w.k_in);
    const dim3 grid((unsigned)gx, (unsigned)gy);
    const bool dyf16 = dyt == RQ_F16, dxf16 = dxt == RQ_F16;
    if (w.format == RQ_Q_ROWWISE_I8)
        return dyf16 ? launch_fmt<RQ_Q_ROWWISE_I8, true>(w, dy, dx, dxf16, m, grid, s)
                     : launch_fmt<RQ_Q_ROWWISE_I8, false>(w, dy, dx, dxf16, m, grid, s);
    return dyf16 ? launch_fmt<RQ_Q_AFFINE_U8, true>(w, dy, dx, dxf16, m, grid, s)
                 : launch_fmt<RQ_Q_AFFINE_U8, false>(w, dy, dx, dxf16, m, grid, s);
}

}  // namespace rq
