// Decode dequant-GEMV for gfx950: Y[m, n] = sum_k X[m, k] * deq(W)[n, k], m <= 16.
//
// Replaces, for one decode token, the reference's f32 `matmul_tiled`
// (rusty-backend/src/kernels.wgsl:7-54) on a load-time-dequantized f32
// weight (kernels.wgsl:379-400): here the int8 codes stream straight from HBM
// (1 B/weight instead of 4 B) and the scale is applied in registers.
//
// Layout and work split (HBM-bound; 1 B of codes per weight):
//  * W is [N, K] row-major int8/uint8, K contiguous, K % 16 == 0, 16-byte
//    aligned rows.  A "chunk" is 16 consecutive codes (one dwordx4).
//  * A block of 256 threads is split into RP = 256/TPR row groups of TPR
//    threads.  Thread tt of a row group owns chunks tt, tt+TPR, ... (< K/16)
//    of every row it visits, so a wave's dwordx4 loads cover 1 KiB of one row
//    contiguously and the lane's X slice (the same K positions for every row)
//    is loaded once and kept in registers as packed fp16.
//  * A block walks `rows_per_block` rows in batches of RB rows per row group;
//    the next batch's codes are loaded before the current batch is reduced.
//  * int8 -> fp16 without a convert: v_perm_b32 places byte b next to 0x64,
//    giving the fp16 value 1024 + b.  Signed codes are first XORed with 0x80
//    (b = q + 128), so the lane computes sum (1152 + q) x with v_dot2_f32_f16
//    and subtracts 1152 * sum x, the lane's own X-slice sum.  Every fp16 value
//    and product is exact; accumulation is f32.
//  * Affine format (reference layout): per chunk the lane applies its group's
//    scale s and bias b: acc += s * sum (1024 + u) x + (b - 1024 s) * sum x.
//  * Wave sums use DPP row operations then two cross-row shuffles; the
//    per-wave totals meet in LDS (one barrier per batch, double-buffered).
//  * f32 activations (the reference's dtype) take the same structure with
//    exact int8 -> f32 conversion and f32 FMAs.
#include "common.hpp"

namespace rq {
namespace {

constexpr int GT = 256;  // threads per block
constexpr int RB = 4;    // rows per batch per row group

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ h2_t as_h2(uint32_t v) { return __builtin_bit_cast(h2_t, v); }

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(as_h2(a), as_h2(b), c, false);
}

// fp16 pairs (1024 + byte0, 1024 + byte1) and (1024 + byte2, 1024 + byte3).
__device__ __forceinline__ uint32_t magic_lo(uint32_t w) { return __builtin_amdgcn_perm(0x64646464u, w, 0x04010400u); }
__device__ __forceinline__ uint32_t magic_hi(uint32_t w) { return __builtin_amdgcn_perm(0x64646464u, w, 0x04030402u); }

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Sum over the 64 lanes of a wave; every lane receives the total.
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp<0x141>(v);  // row_half_mirror
    v += dpp<0x140>(v);  // row_mirror: every lane holds its 16-lane row sum
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 32, 64);
    return v;
}

template <bool XF16> struct XElem;
template <> struct XElem<true> { using T = _Float16; };
template <> struct XElem<false> { using T = float; };

// FMT: 0 = ROWWISE_I8, 1 = AFFINE_U8.  M: max activation rows handled
// (m_act <= M).  CPT: max chunks per thread.  TPR: threads per row group.
template <int M, int CPT, int TPR, int FMT, bool XF16>
__global__ __launch_bounds__(GT) void k_gemv(const uint8_t *__restrict__ W, const float *__restrict__ scales,
                                             const float *__restrict__ biases, const void *__restrict__ Xv,
                                             void *__restrict__ Yv, int y_f16, int m_act, int N, int K,
                                             int group, int rows_per_block) {
    constexpr int RP = GT / TPR;   // row groups per block
    constexpr int WPR = TPR / 64;  // waves per row group
    constexpr int V = RB * M;      // partial sums per thread per batch

    __shared__ float red[2][GT / 64][V];

    const int t = threadIdx.x;
    const int rp = t / TPR, tt = t % TPR;
    const int wave = t / 64, lane = t % 64;
    const int C = K >> 4;

    const int row_begin = blockIdx.x * rows_per_block;
    const int row_end = min(N, row_begin + rows_per_block);

    // ---- batch loader ------------------------------------------------------
    auto load_batch = [&](int base, uint4 (&w)[RB][CPT], float (&sg)[RB][CPT], float (&bg)[RB][CPT]) {
#pragma unroll
        for (int r = 0; r < RB; ++r) {
            const int row = base + r * RP + rp;
#pragma unroll
            for (int j = 0; j < CPT; ++j) {
                const int c = tt + TPR * j;
                const bool ok = row < row_end && c < C;
                const size_t off = (size_t)row * (size_t)K + (size_t)c * 16;
                w[r][j] = ok ? *reinterpret_cast<const uint4 *>(W + off) : make_uint4(0, 0, 0, 0);
                if constexpr (FMT == 1) {
                    const size_t g = off / (size_t)group;
                    sg[r][j] = ok ? scales[g] : 0.0f;
                    bg[r][j] = ok ? (biases ? biases[g] : 0.0f) : 0.0f;
                }
            }
        }
    };

    uint4 wcur[RB][CPT];
    float sgc[RB][CPT], bgc[RB][CPT];
    load_batch(row_begin, wcur, sgc, bgc);

    // ---- X slice ------------------------------------------------------------
    using XT = typename XElem<XF16>::T;
    const XT *X = reinterpret_cast<const XT *>(Xv);
    uint32_t xh[CPT][M][XF16 ? 8 : 1];
    float xf[CPT][M][XF16 ? 1 : 16];
    float xs[CPT][M];
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
        const int c = tt + TPR * j;
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const bool ok = c < C && m < m_act;
            if constexpr (XF16) {
                uint4 a = make_uint4(0, 0, 0, 0), b = make_uint4(0, 0, 0, 0);
                if (ok) {
                    const uint4 *p = reinterpret_cast<const uint4 *>(X + (size_t)m * K + (size_t)c * 16);
                    a = p[0];
                    b = p[1];
                }
                xh[j][m][0] = a.x; xh[j][m][1] = a.y; xh[j][m][2] = a.z; xh[j][m][3] = a.w;
                xh[j][m][4] = b.x; xh[j][m][5] = b.y; xh[j][m][6] = b.z; xh[j][m][7] = b.w;
                float s = 0.0f;
#pragma unroll
                for (int i = 0; i < 8; ++i) s = dot2(xh[j][m][i], 0x3C003C00u, s);  // (1,1) in fp16
                xs[j][m] = s;
            } else {
                float s = 0.0f;
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    xf[j][m][i] = ok ? X[(size_t)m * K + (size_t)c * 16 + i] : 0.0f;
                    s += xf[j][m][i];
                }
                xs[j][m] = s;
            }
        }
    }
    float xs_tot[M];
#pragma unroll
    for (int m = 0; m < M; ++m) {
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < CPT; ++j) s += xs[j][m];
        xs_tot[m] = s;
    }

    int buf = 0;
#pragma unroll 1
    for (int base = row_begin; base < row_end; base += RB * RP) {
        // Scale of the row this thread will store (rowwise format).
        const int st_r = (t / M) % RB, st_m = t % M, st_rp = t / (M * RB);
        const int st_row = base + st_r * RP + st_rp;
        const bool storer = t < RP * RB * M && st_m < m_act && st_row < row_end;
        float st_scale = 1.0f;
        if constexpr (FMT == 0) {
            if (storer) st_scale = scales[st_row];
        }

        // Prefetch the next batch.
        uint4 wnxt[RB][CPT];
        float sgn[RB][CPT], bgn[RB][CPT];
        const bool more = base + RB * RP < row_end;
        if (more) load_batch(base + RB * RP, wnxt, sgn, bgn);

        float acc[RB][M];
#pragma unroll
        for (int r = 0; r < RB; ++r) {
#pragma unroll
            for (int m = 0; m < M; ++m) acc[r][m] = 0.0f;
#pragma unroll
            for (int j = 0; j < CPT; ++j) {
                const uint32_t wd[4] = {wcur[r][j].x, wcur[r][j].y, wcur[r][j].z, wcur[r][j].w};
                if constexpr (XF16) {
                    float d[M];
#pragma unroll
                    for (int m = 0; m < M; ++m) d[m] = 0.0f;
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const uint32_t u = FMT == 0 ? (wd[q] ^ 0x80808080u) : wd[q];
                        const uint32_t lo = magic_lo(u), hi = magic_hi(u);
#pragma unroll
                        for (int m = 0; m < M; ++m) {
                            d[m] = dot2(lo, xh[j][m][2 * q], d[m]);
                            d[m] = dot2(hi, xh[j][m][2 * q + 1], d[m]);
                        }
                    }
#pragma unroll
                    for (int m = 0; m < M; ++m) {
                        if constexpr (FMT == 0) {
                            acc[r][m] += d[m];
                        } else {
                            const float s = sgc[r][j], b = bgc[r][j];
                            acc[r][m] = __builtin_fmaf(s, d[m], acc[r][m]);
                            acc[r][m] = __builtin_fmaf(__builtin_fmaf(-1024.0f, s, b), xs[j][m], acc[r][m]);
                        }
                    }
                } else {
                    float d[M];
#pragma unroll
                    for (int m = 0; m < M; ++m) d[m] = 0.0f;
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const uint32_t byte = (wd[q] >> (8 * e)) & 0xFFu;
                            const float wv = FMT == 0 ? (float)(int8_t)byte : (float)byte;
#pragma unroll
                            for (int m = 0; m < M; ++m) d[m] = __builtin_fmaf(wv, xf[j][m][4 * q + e], d[m]);
                        }
                    }
#pragma unroll
                    for (int m = 0; m < M; ++m) {
                        if constexpr (FMT == 0) {
                            acc[r][m] += d[m];
                        } else {
                            acc[r][m] = __builtin_fmaf(sgc[r][j], d[m], acc[r][m]);
                            acc[r][m] = __builtin_fmaf(bgc[r][j], xs[j][m], acc[r][m]);
                        }
                    }
                }
            }
            if constexpr (FMT == 0 && XF16) {
#pragma unroll
                for (int m = 0; m < M; ++m) acc[r][m] = __builtin_fmaf(-1152.0f, xs_tot[m], acc[r][m]);
            }
        }

        // Wave sums, then across the WPR waves of each row group.
#pragma unroll
        for (int r = 0; r < RB; ++r)
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const float v = wave_sum(acc[r][m]);
                if (lane == 0) red[buf][wave][r * M + m] = v;
            }
        __syncthreads();
        if (storer) {
            float v = 0.0f;
#pragma unroll
            for (int w = 0; w < WPR; ++w) v += red[buf][st_rp * WPR + w][st_r * M + st_m];
            v *= st_scale;
            const size_t o = (size_t)st_m * (size_t)N + (size_t)st_row;
            if (y_f16) reinterpret_cast<_Float16 *>(Yv)[o] = (_Float16)v;
            else reinterpret_cast<float *>(Yv)[o] = v;
        }
        buf ^= 1;

        if (more) {
#pragma unroll
            for (int r = 0; r < RB; ++r)
#pragma unroll
                for (int j = 0; j < CPT; ++j) {
                    wcur[r][j] = wnxt[r][j];
                    sgc[r][j] = sgn[r][j];
                    bgc[r][j] = bgn[r][j];
                }
        }
    }
}

using GemvFn = void (*)(const uint8_t *, const float *, const float *, const void *, void *, int, int, int, int, int,
                        int);

// Instantiated variants: the register-resident X slice must fit without
// spilling (f32 slices are twice the size of fp16 ones).
template <int M, int CPT, int FMT, bool XF16>
constexpr bool kServed = XF16 ? !(M == 8 && CPT == 4 && FMT == 1) : (M * CPT <= 8);

template <int M, int CPT, int TPR, int FMT, bool XF16>
GemvFn one() {
    if constexpr (kServed<M, CPT, FMT, XF16>) return &k_gemv<M, CPT, TPR, FMT, XF16>;
    else return nullptr;
}

template <int M, int CPT, int TPR>
GemvFn pick_fmt(int fmt, bool xf16) {
    if (fmt == 0) return xf16 ? one<M, CPT, TPR, 0, true>() : one<M, CPT, TPR, 0, false>();
    return xf16 ? one<M, CPT, TPR, 1, true>() : one<M, CPT, TPR, 1, false>();
}

template <int M, int CPT>
GemvFn pick_tpr(int tpr, int fmt, bool xf16) {
    switch (tpr) {
    case 64: return pick_fmt<M, CPT, 64>(fmt, xf16);
    case 128: return pick_fmt<M, CPT, 128>(fmt, xf16);
    default: return pick_fmt<M, CPT, 256>(fmt, xf16);
    }
}

template <int M>
GemvFn pick_cpt(int cpt, int tpr, int fmt, bool xf16) {
    switch (cpt) {
    case 1: return pick_tpr<M, 1>(tpr, fmt, xf16);
    case 2: return pick_tpr<M, 2>(tpr, fmt, xf16);
    default: return pick_tpr<M, 4>(tpr, fmt, xf16);
    }
}

}  // namespace

// Returns RQ_UNSUPPORTED (without launching) when the shape or alignment is
// outside what k_gemv serves; the caller then uses the generic kernel.
int launch_gemv(const rq_qweight &w, const void *x, rq_dtype xt, void *y, rq_dtype yt, int m, int num_cus,
                hipStream_t s) {
    const int64_t N = w.n_out, K = w.k_in;
    const bool xf16 = xt == RQ_F16;
    if (K % 16 != 0 || K > 16 * 256 * 4 || N > 0x7fffffff || !aligned(w.codes, 16) ||
        !aligned(x, 16) || (w.format == RQ_Q_AFFINE_U8 && w.group % 16 != 0))
        return RQ_ERR_UNSUPPORTED;
    const int C = (int)(K / 16);
    int tpr = C <= 64 ? 64 : (C <= 128 ? 128 : 256);
    int cpt = (int)cdiv(C, tpr);
    if (cpt == 3) cpt = 4;
    if (cpt > 4) return RQ_ERR_UNSUPPORTED;
    int mt = m <= 1 ? 1 : (m <= 2 ? 2 : (m <= 4 ? 4 : (m <= 8 ? 8 : 16)));
    if (mt == 16) return RQ_ERR_UNSUPPORTED;

    GemvFn fn = nullptr;
    switch (mt) {
    case 1: fn = pick_cpt<1>(cpt, tpr, w.format, xf16); break;
    case 2: fn = pick_cpt<2>(cpt, tpr, w.format, xf16); break;
    case 4: fn = pick_cpt<4>(cpt, tpr, w.format, xf16); break;
    default: fn = pick_cpt<8>(cpt, tpr, w.format, xf16); break;
    }
    if (!fn) return RQ_ERR_UNSUPPORTED;
    const int rp = GT / tpr;
    const int batch_rows = RB * rp;
    // Aim for ~4 resident blocks per CU; at least one batch per block.
    int64_t blocks_target = (int64_t)num_cus * 4;
    int64_t rows_per_block = cdiv(cdiv(N, blocks_target), batch_rows) * batch_rows;
    if (rows_per_block < batch_rows) rows_per_block = batch_rows;
    const int64_t blocks = cdiv(N, rows_per_block);
    hipLaunchKernelGGL(fn, dim3((unsigned)blocks), dim3(GT), 0, s, (const uint8_t *)w.codes, w.scales, w.biases, x,
                       y, yt == RQ_F16 ? 1 : 0, m, (int)N, (int)K, w.group, (int)rows_per_block);
    RQ_LAUNCH_CHECK();
    return RQ_OK;
}

}  // namespace rq
