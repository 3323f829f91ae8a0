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
#include <type_traits>

#include "common.hpp"

namespace rq {
namespace {

constexpr int BM = 64, BN = 64, BK = 32, TH = 256;

// The dequantized value of code c with its row's (per-row codes) or group's
// (affine) scale s and bias b.
template <int FMT>
__device__ __forceinline__ float deq1(uint32_t c, float s, float b) {
    if constexpr (FMT == RQ_Q_ROWWISE_I8) {
        return (float)(int8_t)c * s;
    } else {
        float v;
        {
#pragma clang fp contract(off)
            v = (float)c * s;
            v = v + b;
        }
        return v;
    }
}

// VW: codes 8-byte aligned and k_in % 8 == 0 (8 codes per load).
template <int FMT, bool DYF16, bool DXF16, bool VW>
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

    // raw loads (an out-of-range element loads element 0 of its operand) and
    // the zeroing of out-of-range elements at staging: a branch or a select
    // right after each load made the compiler wait for it before the fmas
    // raw loads into registers (conversions wait for their loads, so they are
    // done when staging): dY values as stored, 8 codes as one 8-byte word (or
    // 8 bytes where codes are unaligned or k_in % 8 != 0), their scales
    typedef _Float16 yt_t;
    std::conditional_t<DYF16, yt_t, float> yr[8];
    uint2 wq;        // VW
    uint8_t wb8[8];  // !VW
    float ws[FMT == RQ_Q_ROWWISE_I8 ? 1 : 8], wb[FMT == RQ_Q_ROWWISE_I8 ? 1 : 8];  // scales (and biases)
    auto load = [&](int64_t k0) {
        const int64_t gr = m0 + ar;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int64_t gc = k0 + ac + e;
            const int64_t o = gr < m && gc < n_out ? gr * n_out + gc : 0;
            if constexpr (DYF16) yr[e] = static_cast<const _Float16 *>(dyv)[o];
            else yr[e] = static_cast<const float *>(dyv)[o];
        }
        const int64_t row = k0 + br, col = c0 + bc;
        if constexpr (VW) {  // k_in % 8 == 0: a thread's 8 columns are all in the row or all past it
            wq = *reinterpret_cast<const uint2 *>(codes + (row < n_out && col < k_in ? row * k_in + col : 0));
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) wb8[e] = codes[row < n_out && col + e < k_in ? row * k_in + col + e : 0];
        }
        if constexpr (FMT == RQ_Q_ROWWISE_I8) {
            ws[0] = scales[row < n_out ? row : 0];
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int64_t g = row < n_out && col + e < k_in ? (row * k_in + col + e) / group : 0;
                ws[e] = scales[g];
                wb[e] = biases ? biases[g] : 0.0f;
            }
        }
    };
    auto stage = [&](int64_t k0) {
        const int64_t gr = m0 + ar;
#pragma unroll
        for (int e = 0; e < 8; ++e) As[ac + e][ar] = gr < m && k0 + ac + e < n_out ? (float)yr[e] : 0.0f;
        const int64_t row = k0 + br, col = c0 + bc;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            uint32_t c;
            if constexpr (VW) c = ((e < 4 ? wq.x : wq.y) >> (8 * (e % 4))) & 0xFFu;
            else c = wb8[e];
            Bs[br][bc + e] = row < n_out && col + e < k_in
                                 ? deq1<FMT>(c, ws[FMT == RQ_Q_ROWWISE_I8 ? 0 : e], wb[FMT == RQ_Q_ROWWISE_I8 ? 0 : e])
                                 : 0.0f;
        }
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
        // the LDS values of step kk + 2 are requested before step kk's fmas
        // (three register sets, the loop fully unrolled)
        float av[3][4], bv[3][4];
        auto rd = [&](int st, int kk) {
#pragma unroll
            for (int i = 0; i < 4; ++i) av[st][i] = As[kk][ty + 16 * i];
#pragma unroll
            for (int j = 0; j < 4; ++j) bv[st][j] = Bs[kk][tx + 16 * j];
        };
        rd(0, 0);
        rd(1, 1);
#pragma unroll
        for (int kk = 0; kk < BK; ++kk) {
            if (kk + 2 < BK) rd((kk + 2) % 3, kk + 2);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_fmaf(av[kk % 3][i], bv[kk % 3][j], acc[i][j]);
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
    const bool vw = w.k_in % 8 == 0 && aligned(codes, 8);
    auto go = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, grid, dim3(TH), 0, s, codes, w.scales, w.biases, w.group, dy, dx, m, w.n_out,
                           w.k_in);
    };
    if (dxf16) vw ? go(k_qmatmul_dx<FMT, DYF16, true, true>) : go(k_qmatmul_dx<FMT, DYF16, true, false>);
    else vw ? go(k_qmatmul_dx<FMT, DYF16, false, true>) : go(k_qmatmul_dx<FMT, DYF16, false, false>);
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
