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
#include <algorithm>
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

// ---- Input gradient on the matrix cores (per-row int8 codes) ----
//
// dX[m][k] = sum_n dY[m][n] s[n] q[n][k] is a GEMM whose reduction runs along
// n_out, while the int8 rows of W are contiguous along k_in: the matrix cores
// need the reduction contiguous in each lane's operand.  So a table built once
// per weight (load time, rq_qweight_dx_table) holds the codes transposed and
// written twice side by side, qt[k][j] = q[j mod n][k] for j < 2 n_out, and
// k_in unit scales; each dY row becomes v = dY s (f32, one rounding) scaled by
// the power of two 2^-e that puts max |v| in [2^14, 2^15), then two fp16
// halves x2[m] = [fp16(v 2^-e) | fp16(v 2^-e - hi)] (hi + lo = v 2^-e to
// ~2^-22 relative).  The prefill GEMM (gemm.hip) then computes
// dX[m][k] = 2^e sum_j x2[m][j] qt[k][j]: exact fp16 x int8 products, f32
// sums -- the f32 bar against the exact product, not the chain's bit pattern
// (rq_qmatmul_dx keeps that).  Memory: the table is 2 B per weight element.
namespace rq {
namespace {

constexpr int TT = 64;  // transpose tile, bytes per side

// qt[k][j] = qt[k][j + n] = q[j][k], one 64 x 64 tile per block; n % 16 == 0,
// k % 16 == 0, so every 16-byte piece lies wholly inside or outside.
__global__ __launch_bounds__(256) void k_dx_transpose(const uint8_t *__restrict__ q, uint8_t *__restrict__ qt,
                                                      int64_t n, int64_t k) {
    __shared__ uint8_t tile[TT][TT + 4];  // [n local][k local]
    const int t = threadIdx.x, r = t / 4, c = (t % 4) * 16;
    const int64_t n0 = (int64_t)blockIdx.y * TT, k0 = (int64_t)blockIdx.x * TT;
    {
        const int64_t gn = n0 + r, gk = k0 + c;
        const uint4 v = gn < n && gk < k ? *reinterpret_cast<const uint4 *>(q + gn * k + gk) : make_uint4(0, 0, 0, 0);
        const uint32_t wd[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int e = 0; e < 16; ++e) tile[r][c + e] = (uint8_t)(wd[e / 4] >> (8 * (e % 4)));
    }
    __syncthreads();
    const int64_t gk = k0 + r, gn = n0 + c;  // row gk of qt, its bytes gn .. gn + 15
    if (gk < k && gn < n) {
        uint32_t wd[4] = {0, 0, 0, 0};
#pragma unroll
        for (int e = 0; e < 16; ++e) wd[e / 4] |= (uint32_t)tile[c + e][r] << (8 * (e % 4));
        const uint4 v = make_uint4(wd[0], wd[1], wd[2], wd[3]);
        *reinterpret_cast<uint4 *>(qt + gk * 2 * n + gn) = v;
        *reinterpret_cast<uint4 *>(qt + gk * 2 * n + n + gn) = v;
    }
}

__global__ __launch_bounds__(256) void k_fill_ones(float *__restrict__ p, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) p[i] = 1.0f;
}

template <int CTRL>
__device__ __forceinline__ float dppf(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));

// Row i of dY (one block): v[j] = dY[i][j] s[j]; the row maximum (DPP steps
// and one barrier), 2^e with max |v| 2^-e in [2^14, 2^15) (e >= -126: 2^e
// stays a normal f32; a zero row gives e = 0), then x2[i][j] = hi,
// x2[i][n + j] = lo and xs[i] = 2^e.  Pieces of 8 values (n % 8 == 0): with
// VEC (dY and s 16-byte aligned) 16- or 32-byte loads, and with NI > 0
// (n <= 2048 NI) each thread keeps its NI pieces in registers from the
// maximum to the split, so the row is read once; otherwise it is read twice
// (the second time from L2).
template <bool DYF16, bool VEC, int NI>
__global__ __launch_bounds__(256) void k_dx_split(const void *__restrict__ dy, const float *__restrict__ s,
                                                  _Float16 *__restrict__ x2, float *__restrict__ xs, int64_t n) {
    __shared__ float wmax[4];
    const int64_t row = blockIdx.x;
    const int t = threadIdx.x, lane = t & 63;
    const int n8 = (int)(n / 8);
    auto piece = [&](int i, float *v) {  // v = dY[row][8i + e] * s[8i + e]
        float sv[8], dv[8];
        if constexpr (VEC) {
            const float4 s0 = reinterpret_cast<const float4 *>(s)[2 * i], s1 = reinterpret_cast<const float4 *>(s)[2 * i + 1];
            sv[0] = s0.x; sv[1] = s0.y; sv[2] = s0.z; sv[3] = s0.w; sv[4] = s1.x; sv[5] = s1.y; sv[6] = s1.z; sv[7] = s1.w;
            if constexpr (DYF16) {
                const half8_t h = reinterpret_cast<const half8_t *>(static_cast<const _Float16 *>(dy) + row * n)[i];
#pragma unroll
                for (int e = 0; e < 8; ++e) dv[e] = (float)h[e];
            } else {
                const float4 *d4 = reinterpret_cast<const float4 *>(static_cast<const float *>(dy) + row * n);
                const float4 a = d4[2 * i], b = d4[2 * i + 1];
                dv[0] = a.x; dv[1] = a.y; dv[2] = a.z; dv[3] = a.w; dv[4] = b.x; dv[5] = b.y; dv[6] = b.z; dv[7] = b.w;
            }
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int64_t j = (int64_t)8 * i + e;
                sv[e] = s[j];
                dv[e] = DYF16 ? (float)static_cast<const _Float16 *>(dy)[row * n + j]
                              : static_cast<const float *>(dy)[row * n + j];
            }
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = dv[e] * sv[e];
    };
    auto amax8 = [](const float *v) {
        float a = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) a = fmaxf(a, fabsf(v[e]));
        return a;
    };
    float amax = 0.0f;
    float held[NI > 0 ? NI : 1][8];
    if constexpr (NI > 0) {
#pragma unroll
        for (int j = 0; j < NI; ++j) {  // every load in flight before the first use
            const int i = t + 256 * j;
            if (i < n8) piece(i, held[j]);
            else
#pragma unroll
                for (int e = 0; e < 8; ++e) held[j][e] = 0.0f;
        }
#pragma unroll
        for (int j = 0; j < NI; ++j) amax = fmaxf(amax, amax8(held[j]));
    } else {
        for (int i = t; i < n8; i += 256) {
            float v[8];
            piece(i, v);
            amax = fmaxf(amax, amax8(v));
        }
    }
    amax = fmaxf(amax, dppf<0xB1>(amax));   // quad_perm [1,0,3,2]
    amax = fmaxf(amax, dppf<0x4E>(amax));   // quad_perm [2,3,0,1]
    amax = fmaxf(amax, dppf<0x141>(amax));  // row_half_mirror
    amax = fmaxf(amax, dppf<0x140>(amax));  // row_mirror: each 16-lane row holds its maximum
    const auto rl = [](float v, int l) {
        return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
    };
    amax = fmaxf(fmaxf(rl(amax, 0), rl(amax, 16)), fmaxf(rl(amax, 32), rl(amax, 48)));
    if (lane == 0) wmax[t >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    const int e = max(__builtin_amdgcn_frexp_expf(amax) - 15, -126);
    half8_t *hr = reinterpret_cast<half8_t *>(x2 + row * 2 * n);
    auto split = [&](int i, const float *v) {
        half8_t hi, lo;
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const float w = __builtin_amdgcn_ldexpf(v[q], -e);
            hi[q] = (_Float16)w;
            lo[q] = (_Float16)(w - (float)hi[q]);
        }
        hr[i] = hi;
        hr[n8 + i] = lo;
    };
    if constexpr (NI > 0) {
#pragma unroll
        for (int j = 0; j < NI; ++j) {
            const int i = t + 256 * j;
            if (i < n8) split(i, held[j]);
        }
    } else {
        for (int i = t; i < n8; i += 256) {
            float v[8];
            piece(i, v);
            split(i, v);
        }
    }
    if (t == 0) xs[row] = __builtin_amdgcn_ldexpf(1.0f, e);
}

bool dx_table_ok(const rq_qweight &w) {
    return w.format == RQ_Q_ROWWISE_I8 && w.n_out >= 32 && w.n_out % 32 == 0 && w.k_in >= 16 && w.k_in % 16 == 0 &&
           2 * w.n_out <= (1 << 21) && w.k_in <= 0x7fffffff && aligned(w.codes, 16);
}
size_t dx_codes_bytes(const rq_qweight &w) { return ((size_t)2 * w.n_out * w.k_in + 255) & ~size_t(255); }

}  // namespace
}  // namespace rq

using namespace rq;

extern "C" {

size_t rq_qweight_dx_table_bytes(const rq_qweight *w) {
    if (!w || check_qweight(w) != RQ_OK || !dx_table_ok(*w)) return 0;
    return dx_codes_bytes(*w) + (size_t)w->k_in * 4;
}

int rq_qweight_dx_table(rq_ctx *ctx, const rq_qweight *w, void *table, size_t table_bytes, rq_stream stream) {
    RQ_ENTER(ctx);
    int st = check_qweight(w);
    if (st != RQ_OK) return st;
    if (!dx_table_ok(*w))
        return fail(RQ_ERR_UNSUPPORTED, "the matrix-core input gradient takes per-row int8 codes, 16-byte aligned, "
                                        "n_out a multiple of 32, k_in a multiple of 16");
    const size_t need = rq_qweight_dx_table_bytes(w);
    if (!table || table_bytes < need || !aligned(table, 256))
        return fail(RQ_ERR_INVALID_ARGUMENT, "table of %zu bytes (256-byte aligned), %zu needed", table_bytes, need);
    hipStream_t s = pick(ctx, stream);
    const int64_t n = w->n_out, k = w->k_in;
    if (cdiv(k, TT) > 0x7fffffff || cdiv(n, TT) > 65535) return fail(RQ_ERR_SHAPE, "weight too large to transpose");
    uint8_t *qt = static_cast<uint8_t *>(table);
    hipLaunchKernelGGL(k_dx_transpose, dim3((unsigned)cdiv(k, TT), (unsigned)cdiv(n, TT)), dim3(256), 0, s,
                       static_cast<const uint8_t *>(w->codes), qt, n, k);
    RQ_LAUNCH_CHECK();
    float *ones = reinterpret_cast<float *>(qt + dx_codes_bytes(*w));
    hipLaunchKernelGGL(k_fill_ones, dim3((unsigned)std::min<int64_t>(cdiv(k, 256), 4096)), dim3(256), 0, s, ones, k);
    RQ_LAUNCH_CHECK();
    return RQ_OK;
}

size_t rq_qmatmul_dx_mfma_workspace(int64_t m, int64_t n_out) {
    if (m < 0 || n_out < 0) return 0;
    return (((size_t)m * (size_t)n_out * 4 + 255) & ~size_t(255)) + (size_t)m * 4;
}

int rq_qmatmul_dx_mfma(rq_ctx *ctx, const rq_qweight *w, const void *table, const void *dy, rq_dtype dy_dtype,
                       void *dx, rq_dtype dx_dtype, int64_t m, void *workspace, size_t workspace_bytes,
                       rq_stream stream) {
    RQ_ENTER(ctx);
    int st = check_qweight(w);
    if (st != RQ_OK) return st;
    if ((dy_dtype != RQ_F16 && dy_dtype != RQ_F32) || (dx_dtype != RQ_F16 && dx_dtype != RQ_F32))
        return fail(RQ_ERR_INVALID_ARGUMENT, "dtype must be RQ_F16 or RQ_F32");
    if (!dx_table_ok(*w))
        return fail(RQ_ERR_UNSUPPORTED, "the matrix-core input gradient takes per-row int8 codes, 16-byte aligned, "
                                        "n_out a multiple of 32, k_in a multiple of 16");
    if (m < 0) return fail(RQ_ERR_SHAPE, "negative m");
    int64_t t;
    if (!mul_ok(m, w->k_in, &t) || !mul_ok(m, 2 * w->n_out, &t) || m > 0x7fffffff)
        return fail(RQ_ERR_SHAPE, "shape overflows");
    if (m == 0) return RQ_OK;
    if (!dx || !dy || !table) return fail(RQ_ERR_INVALID_ARGUMENT, "null gradient or table pointer");
    if (!aligned(table, 256)) return fail(RQ_ERR_INVALID_ARGUMENT, "table must be 256-byte aligned");
    const size_t need = rq_qmatmul_dx_mfma_workspace(m, w->n_out);
    if (!workspace || workspace_bytes < need || !aligned(workspace, 256))
        return fail(RQ_ERR_INVALID_ARGUMENT, "workspace of %zu bytes (256-byte aligned), %zu needed",
                    workspace_bytes, need);
    hipStream_t s = pick(ctx, stream);
    const int64_t n = w->n_out, k = w->k_in;
    _Float16 *x2 = static_cast<_Float16 *>(workspace);
    float *xs = reinterpret_cast<float *>(static_cast<char *>(workspace) + (((size_t)m * n * 4 + 255) & ~size_t(255)));
    {
        const bool vec = aligned(dy, 16) && aligned(w->scales, 16);
        const int64_t per = cdiv(n / 8, 256);  // 8-value pieces per thread
        auto go = [&](auto f16, auto v, auto ni) {
            hipLaunchKernelGGL((k_dx_split<decltype(f16)::value, decltype(v)::value, decltype(ni)::value>),
                               dim3((unsigned)m), dim3(256), 0, s, dy, w->scales, x2, xs, n);
        };
        auto by_ni = [&](auto f16, auto v) {
            if (per <= 1) go(f16, v, std::integral_constant<int, 1>{});
            else if (per <= 2) go(f16, v, std::integral_constant<int, 2>{});
            else if (per <= 4) go(f16, v, std::integral_constant<int, 4>{});
            else go(f16, v, std::integral_constant<int, 0>{});
        };
        auto by_vec = [&](auto f16) {
            if (vec) by_ni(f16, std::true_type{});
            else by_ni(f16, std::false_type{});
        };
        if (dy_dtype == RQ_F16) by_vec(std::true_type{});
        else by_vec(std::false_type{});
        RQ_LAUNCH_CHECK();
    }
    // the transposed problem: k_in rows of 2 n_out codes, unit scales
    const uint8_t *qt = static_cast<const uint8_t *>(table);
    const rq_qweight wt{qt, reinterpret_cast<const float *>(qt + dx_codes_bytes(*w)), nullptr, k, 2 * n,
                        RQ_Q_ROWWISE_I8, 0, nullptr};
    st = launch_gemm_f16_scaled(wt, wt.scales, x2, xs, dx, dx_dtype, m, ctx->num_cus, gemm_workspace(ctx, s), s);
    if (st == RQ_ERR_UNSUPPORTED) return fail(st, "dx pointer alignment (8 bytes fp16, 16 bytes f32) not met");
    return st;
}

}  // extern "C"
