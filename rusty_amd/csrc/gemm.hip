// Prefill dequant-GEMM for gfx950: Y[m, n] = s[n] * sum_k X[m, k] * q[n, k].
//
// Replaces, for a prompt of many tokens, the reference's f32 `matmul_tiled`
// (rusty-backend/src/kernels.wgsl:7-54) on a load-time-dequantized weight
// (kernels.wgsl:379-400).  MFMA-bound: 2*M*N*K flops over 1 B/weight + 2 B/act.
//
//  * Block tile 128 (X rows) x 128 (W rows) x 64 (k), 256 threads = 4 waves
//    in a 2x2 grid, each wave 64x64 = 4x4 tiles of v_mfma_f32_16x16x32_f16
//    with f32 accumulators.
//  * Operands: MFMA A = W (16 output features x 32 k), B = X^T (32 k x 16
//    tokens).  The f32 result of a tile then sits as 4 consecutive features of
//    one token per lane, so the epilogue stores 8 B (fp16) per lane.
//  * Staging: global -> registers -> LDS, double-buffered, one barrier per
//    k-tile; the next tile's global loads are in flight while the current
//    tile is multiplied.  LDS rows are padded (X: 144 B, W: 72 B) so the
//    16 rows read by one MFMA operand fall in distinct banks.
//  * int8 stays int8 in LDS (half the bytes of fp16) and is expanded right
//    before the MFMA: XOR 0x80 turns q into q+128, v_perm_b32 builds fp16
//    1024 + (q+128) = 1152 + q, v_pk_add_f16 subtracts 1152.  Exact.
//  * Epilogue: per-feature scale (f32), convert, store.
#include "common.hpp"

namespace rq {
namespace {

constexpr int BM = 128, BN = 128, BK = 64, TH = 256;
constexpr int XS_STRIDE = BK * 2 + 16;  // bytes per X row in LDS
constexpr int WS_STRIDE = BK + 8;       // bytes per W row in LDS
constexpr int XS_BYTES = BM * XS_STRIDE;
constexpr int WS_BYTES = BN * WS_STRIDE;

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t i8x2_to_f16x2(uint32_t u, uint32_t sel) {
    const uint32_t m = __builtin_amdgcn_perm(0x64646464u, u, sel);
    const h2_t v = __builtin_bit_cast(h2_t, m) - (h2_t){(_Float16)1152.0f, (_Float16)1152.0f};
    return __builtin_bit_cast(uint32_t, v);
}

// 8 signed int8 codes (two dwords) -> 8 exact fp16 values.
__device__ __forceinline__ half8 i8x8_to_half8(uint2 w) {
    const uint32_t a = w.x ^ 0x80808080u, b = w.y ^ 0x80808080u;
    uint4 r;
    r.x = i8x2_to_f16x2(a, 0x04010400u);
    r.y = i8x2_to_f16x2(a, 0x04030402u);
    r.z = i8x2_to_f16x2(b, 0x04010400u);
    r.w = i8x2_to_f16x2(b, 0x04030402u);
    return __builtin_bit_cast(half8, r);
}

__global__ __launch_bounds__(TH) void k_gemm_rowwise(const int8_t *__restrict__ W, const float *__restrict__ scales,
                                                     const _Float16 *__restrict__ X, void *__restrict__ Yv,
                                                     int y_f16, int M, int N, int K) {
    __shared__ __attribute__((aligned(16))) uint8_t lds[2 * (XS_BYTES + WS_BYTES)];

    const int t = threadIdx.x;
    const int wave = t / 64, lane = t % 64;
    const int wm = wave / 2, wn = wave % 2;  // wave tile: rows wm*64 of X, wn*64 of W
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;

    // global -> register mapping
    // X tile 128 x 64 fp16: thread covers rows t/8 + 32p (p<4), 16 B at col (t%8)*8
    // W tile 128 x 64 i8  : thread covers rows t/4 + 64p (p<2), 16 B at col (t%4)*16
    const int xr = t / 8, xc = (t % 8) * 8;
    const int wr = t / 4, wc = (t % 4) * 16;

    uint4 xreg[4], wreg[2];
    auto gload = [&](int k0) {
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const int row = m0 + xr + 32 * p;
            xreg[p] = row < M ? *reinterpret_cast<const uint4 *>(X + (size_t)row * K + k0 + xc) : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            const int row = n0 + wr + 64 * p;
            wreg[p] = row < N ? *reinterpret_cast<const uint4 *>(W + (size_t)row * K + k0 + wc) : make_uint4(0, 0, 0, 0);
        }
    };
    auto lstore = [&](int buf) {
        uint8_t *xs = lds + buf * (XS_BYTES + WS_BYTES);
        uint8_t *ws = xs + XS_BYTES;
#pragma unroll
        for (int p = 0; p < 4; ++p) *reinterpret_cast<uint4 *>(xs + (xr + 32 * p) * XS_STRIDE + xc * 2) = xreg[p];
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            // W rows are 72 B apart: 8-byte aligned only, store as two halves.
            uint2 *d = reinterpret_cast<uint2 *>(ws + (wr + 64 * p) * WS_STRIDE + wc);
            d[0] = make_uint2(wreg[p].x, wreg[p].y);
            d[1] = make_uint2(wreg[p].z, wreg[p].w);
        }
    };

    floatx4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = (floatx4){0.0f, 0.0f, 0.0f, 0.0f};

    const int nk = K / BK;
    gload(0);
    lstore(0);
    __syncthreads();

    const int fr = lane % 16;        // operand row within a 16-row tile
    const int fk = (lane / 16) * 8;  // first of the lane's 8 k values within a 32-k step

#pragma unroll 1
    for (int kt = 0; kt < nk; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < nk) gload((kt + 1) * BK);
        const uint8_t *xs = lds + buf * (XS_BYTES + WS_BYTES);
        const uint8_t *ws = xs + XS_BYTES;
#pragma unroll
        for (int ks = 0; ks < BK; ks += 32) {
            half8 a[4], b[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint2 wv = *reinterpret_cast<const uint2 *>(ws + (wn * 64 + i * 16 + fr) * WS_STRIDE + ks + fk);
                a[i] = i8x8_to_half8(wv);
            }
#pragma unroll
            for (int j = 0; j < 4; ++j)
                b[j] = *reinterpret_cast<const half8 *>(xs + (wm * 64 + j * 16 + fr) * XS_STRIDE + (ks + fk) * 2);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i], b[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < nk) lstore(buf ^ 1);
        __syncthreads();
    }

    // Epilogue: acc[i][j] holds D[feature = 4*(lane/16) + r][token = lane%16]
    // of tile (features n0 + wn*64 + 16 i, tokens m0 + wm*64 + 16 j).
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int nb = n0 + wn * 64 + i * 16 + (lane / 16) * 4;
        float sc[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) sc[r] = nb + r < N ? scales[nb + r] : 0.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int mm = m0 + wm * 64 + j * 16 + fr;
            if (mm >= M) continue;
            float v[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) v[r] = acc[i][j][r] * sc[r];
            const size_t o = (size_t)mm * N + nb;
            if (nb + 4 <= N && (N % 4) == 0) {
                if (y_f16) {
                    h2_t lo = {(_Float16)v[0], (_Float16)v[1]}, hi = {(_Float16)v[2], (_Float16)v[3]};
                    uint2 pk = make_uint2(__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi));
                    *reinterpret_cast<uint2 *>(reinterpret_cast<_Float16 *>(Yv) + o) = pk;
                } else {
                    *reinterpret_cast<float4 *>(reinterpret_cast<float *>(Yv) + o) = make_float4(v[0], v[1], v[2], v[3]);
                }
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    if (nb + r >= N) break;
                    if (y_f16) reinterpret_cast<_Float16 *>(Yv)[o + r] = (_Float16)v[r];
                    else reinterpret_cast<float *>(Yv)[o + r] = v[r];
                }
            }
        }
    }
}

}  // namespace

// Returns RQ_ERR_UNSUPPORTED (without launching) outside what k_gemm_rowwise
// serves; the caller then uses the generic kernel.
int launch_gemm(const rq_qweight &w, const void *x, rq_dtype xt, void *y, rq_dtype yt, int64_t m, int num_cus,
                hipStream_t s) {
    (void)num_cus;
    const int64_t N = w.n_out, K = w.k_in;
    if (w.format != RQ_Q_ROWWISE_I8 || xt != RQ_F16 || K % BK != 0 || !aligned(w.codes, 16) || !aligned(x, 16) ||
        m > 0x7fffffff || N > 0x7fffffff || cdiv(m, BM) > 65535)
        return RQ_ERR_UNSUPPORTED;
    if (yt == RQ_F16 ? !aligned(y, 8) : !aligned(y, 16)) return RQ_ERR_UNSUPPORTED;
    const dim3 grid((unsigned)cdiv(N, BN), (unsigned)cdiv(m, BM));
    hipLaunchKernelGGL(k_gemm_rowwise, grid, dim3(TH), 0, s, (const int8_t *)w.codes, w.scales,
                       (const _Float16 *)x, y, yt == RQ_F16 ? 1 : 0, (int)m, (int)N, (int)K);
    RQ_LAUNCH_CHECK();
    return RQ_OK;
}

}  // namespace rq
