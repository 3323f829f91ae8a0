// Decode dequant-GEMV on the matrix cores, 5 <= m <= 16 tokens:
// Y[m, n] = s[n] * sum_k X[m, k] * q[n, k].
//
// Still HBM-bound (every weight byte read once) but with 5-16 activation rows
// the per-byte arithmetic no longer fits the VALU budget of the dot2 kernel,
// so the products go to v_mfma_f32_16x16x32_f16 (16 features x 16 tokens x 32
// k per instruction; MFMA throughput is far from the limit here):
//  * One block of 4 waves per 16 output features; the waves split K into
//    steps of 256 (step s goes to wave s % 4).  Per step a wave moves its
//    weight (16 rows x 256 B) and activations (16 tokens x 256 fp16) with
//    direct-to-LDS DMA in 1 KiB units of contiguous row runs -- the access
//    pattern that streams at full rate -- and reads them back in MFMA
//    layout.  Both LDS copies are XOR-swizzled per 16-byte chunk (chunk c of
//    row r at c ^ r), so the 16 rows an MFMA operand reads fall in distinct
//    banks.  Tokens >= m, rows >= N and k >= K read as zero.
//  * Three steps per wave are in flight (a 3-buffer LDS ring per wave); the
//    loop issues no compiler-visible global load, so its only vector-memory
//    waits are the explicit vmcnt counts on the wave's own DMA, and there is
//    no block barrier inside the K loop.
//  * The weight is expanded exactly in registers: XOR 0x80, v_perm_b32 under
//    exponent 0x64 (fp16 1152+q), v_pk_add_f16 -1152.
//  * The four waves' 16x16 partial sums meet in LDS once; scale, fp16/f32 store.
#include "common.hpp"

namespace rq {
namespace {

constexpr int TH = 256;
constexpr int FB = 16;                 // features per block
constexpr int KS = 256;                // k per wave per step
constexpr int WSTEP = FB * KS;         // weight bytes per step (4 KiB, 4 DMA units)
constexpr int XSTEP = 16 * KS * 2;     // activation bytes per step (8 KiB, 8 DMA units)
constexpr int NDMA = (WSTEP + XSTEP) / 1024;  // DMA ops per wave per step
constexpr int RING = 3;
constexpr uint32_t kOOB = 0x80000000u;

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), 0, bytes, 0x00020000);
}
// LDS[lds_base + 16 * lane] = buffer[voff] (see gemm.hip: explicit vmcnt waits by the reader).
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, const void *lds_base, uint32_t voff) {
    const uint32_t l = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_void *)lds_base);
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                 :
                 : "s"(l), "v"(voff), "s"(r)
                 : "memory", "m0");
}
// Waits until at most N vector-memory operations of this wave are outstanding
// (they retire in issue order).  Inline asm with a memory clobber, so the
// compiler cannot move LDS reads of the landed data above the wait.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// Waits until every LDS read of this wave has returned its data.
__device__ __forceinline__ void wait_lgkm0() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

__device__ __forceinline__ uint32_t i8x2_to_f16x2(uint32_t u, uint32_t sel) {
    const uint32_t m = __builtin_amdgcn_perm(0x64646464u, u, sel);
    const h2_t v = __builtin_bit_cast(h2_t, m) - (h2_t){(_Float16)1152.0f, (_Float16)1152.0f};
    return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ half8 i8x8_to_half8(uint2 w) {
    const uint32_t a = w.x ^ 0x80808080u, b = w.y ^ 0x80808080u;
    uint4 r;
    r.x = i8x2_to_f16x2(a, 0x04010400u);
    r.y = i8x2_to_f16x2(a, 0x04030402u);
    r.z = i8x2_to_f16x2(b, 0x04010400u);
    r.w = i8x2_to_f16x2(b, 0x04030402u);
    return __builtin_bit_cast(half8, r);
}

struct StepBuf {
    uint8_t w[WSTEP];
    uint8_t x[XSTEP];
};

__device__ __forceinline__ float silu(float v) { return v / (1.0f + expf(-v)); }

// SWI: SwiGLU gate/up pass -- the block's 16 weight rows are 8 gate rows (W)
// and the same 8 rows of the up weight (W2); it writes h = silu(g) * u (fp16).
template <bool SWI>
__global__ __launch_bounds__(TH) void k_gemv_mfma(const int8_t *__restrict__ W, const float *__restrict__ scales,
                                                  const int8_t *__restrict__ W2, const float *__restrict__ scales2,
                                                  const _Float16 *__restrict__ X, void *__restrict__ Yv, int y_f16,
                                                  int m_act, int N, int K) {
    constexpr int RB = SWI ? FB / 2 : FB;  // output rows per block
    __shared__ __attribute__((aligned(1024))) StepBuf ring[4][RING];  // [wave][slot]
    __shared__ floatx4 red[4][64];

    const int t = threadIdx.x, wave = t / 64, lane = t % 64;
    const int n0 = blockIdx.x * RB;
    const int rows_here = min(RB, N - n0);
    const auto rw = make_rsrc(W + (size_t)n0 * K, (uint32_t)rows_here * (uint32_t)K);
    const auto rw2 = make_rsrc((SWI ? W2 : W) + (size_t)n0 * K, (uint32_t)rows_here * (uint32_t)K);
    const auto rx = make_rsrc(X, (uint32_t)m_act * (uint32_t)K * 2u);
    const int nsteps_total = (K + KS - 1) / KS;
    const int my_steps = (nsteps_total - wave + 3) / 4;  // steps wave, wave + 4, ...

    // DMA of one step into ring slot `slot`.  Weight unit u (0..3): rows
    // 4u..4u+3, lane -> row 4u + l/16, slot chunk c = l%16 holds global
    // chunk c ^ row.  Activation unit u (0..7): tokens 2u, 2u+1, lane ->
    // token 2u + l/32, slot chunk c = l%32 holds global chunk c ^ token.
    auto dma_step = [&](int slot, int step) {
        StepBuf &b = ring[wave][slot];
        const int k0 = step * KS;
        const bool live = step < nsteps_total;
#pragma unroll
        for (int u = 0; u < WSTEP / 1024; ++u) {
            const int row = 4 * u + lane / 16, c = lane % 16;
            const int k = k0 + ((c ^ row) & 15) * 16;
            const bool second = SWI && u >= WSTEP / 2048;  // SwiGLU: rows 8..15 come from the up weight
            const uint32_t grow = SWI ? (uint32_t)(row % RB) : (uint32_t)row;
            dma16(second ? rw2 : rw, b.w + u * 1024, (live && k < K) ? grow * K + k : kOOB);
        }
#pragma unroll
        for (int u = 0; u < XSTEP / 1024; ++u) {
            const int tok = 2 * u + lane / 32, c = lane % 32;
            const int k = k0 + ((c ^ tok) & 31) * 8;
            dma16(rx, b.x + u * 1024, (live && k < K) ? ((uint32_t)tok * K + k) * 2u : kOOB);
        }
    };

    floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    const int fr = lane % 16, g = lane / 16;  // MFMA operand row / lane group
    auto mma_step = [&](int slot) {
        const StepBuf &b = ring[wave][slot];
#pragma unroll
        for (int s = 0; s < KS / 32; ++s) {
            // A = weight row fr, k = 32s + 8g .. +8: global chunk 2s + g/2, half g%2
            const int cw = 2 * s + g / 2;
            const uint2 wv = *reinterpret_cast<const uint2 *>(b.w + fr * KS + ((cw ^ fr) & 15) * 16 + (g % 2) * 8);
            // B = activations of token fr, same k: global chunk 4s + g (8 fp16 per chunk)
            const int cx = 4 * s + g;
            const half8 xv = *reinterpret_cast<const half8 *>(b.x + fr * KS * 2 + ((cx ^ fr) & 31) * 16);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(i8x8_to_half8(wv), xv, acc, 0, 0, 0);
        }
    };

    // Ring: steps j, j+1, j+2 in flight; the DMA of steps past this wave's
    // range reads zeros, so every wait has the same count.
#pragma unroll
    for (int j = 0; j < RING; ++j) dma_step(j, wave + 4 * j);
#pragma unroll 1
    for (int j = 0; j < my_steps; j += RING) {
#pragma unroll
        for (int r = 0; r < RING; ++r) {
            if (j + r < my_steps) {
                wait_vmcnt<(RING - 1) * NDMA>();  // step j+r landed
                mma_step(r);
                wait_lgkm0();  // slot fully read before its refill
                dma_step(r, wave + 4 * (j + r + RING));
            }
        }
    }
    wait_vmcnt<0>();  // no DMA in flight past this point

    // acc = D[feature 4*g + r][token fr], partial over this wave's steps.
    red[wave][lane] = acc;
    __syncthreads();
    if (wave == 0) {
        floatx4 v = red[0][lane];
#pragma unroll
        for (int w = 1; w < 4; ++w) {
            const floatx4 o = red[w][lane];
            v[0] += o[0];
            v[1] += o[1];
            v[2] += o[2];
            v[3] += o[3];
        }
        const int m = fr;
        if constexpr (SWI) {
            // gate rows 0..7 sit in lane groups 0-1, up rows 8..15 in groups 2-3
            red[0][lane] = v;
            wait_lgkm0();
            const floatx4 u = red[0][(lane + 32) % 64];
            if (g < 2 && m < m_act) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int f = 4 * g + r;
                    if (f < rows_here) {
                        const float h = silu(v[r] * scales[n0 + f]) * (u[r] * scales2[n0 + f]);
                        reinterpret_cast<_Float16 *>(Yv)[(size_t)m * N + n0 + f] = (_Float16)h;
                    }
                }
            }
        } else if (m < m_act) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int f = 4 * g + r;
                if (f < rows_here) {
                    const float y = v[r] * scales[n0 + f];
                    const size_t o = (size_t)m * N + n0 + f;
                    if (y_f16) reinterpret_cast<_Float16 *>(Yv)[o] = (_Float16)y;
                    else reinterpret_cast<float *>(Yv)[o] = y;
                }
            }
        }
    }
}

}  // namespace

static int launch_mfma(const rq_qweight &w, const rq_qweight *w2, const void *x, void *y, rq_dtype yt, int m,
                       hipStream_t s) {
    const int64_t N = w.n_out, K = w.k_in;
    // 32-bit buffer offsets: 16 activation rows of K fp16 must stay below 2^31 bytes.
    if (w.format != RQ_Q_ROWWISE_I8 || m < 1 || m > 16 || K % 16 != 0 || K > (1 << 24) || N > 0x7fffffff ||
        !aligned(w.codes, 16) || !aligned(x, 16))
        return RQ_ERR_UNSUPPORTED;
    if (w2 && (w2->format != RQ_Q_ROWWISE_I8 || !aligned(w2->codes, 16))) return RQ_ERR_UNSUPPORTED;
    const int64_t blocks = cdiv(N, w2 ? FB / 2 : FB);
    if (w2)
        hipLaunchKernelGGL(k_gemv_mfma<true>, dim3((unsigned)blocks), dim3(TH), 0, s, (const int8_t *)w.codes,
                           w.scales, (const int8_t *)w2->codes, w2->scales, (const _Float16 *)x, y, 1, m, (int)N,
                           (int)K);
    else
        hipLaunchKernelGGL(k_gemv_mfma<false>, dim3((unsigned)blocks), dim3(TH), 0, s, (const int8_t *)w.codes,
                           w.scales, nullptr, nullptr, (const _Float16 *)x, y, yt == RQ_F16 ? 1 : 0, m, (int)N,
                           (int)K);
    RQ_LAUNCH_CHECK();
    return RQ_OK;
}

int launch_gemv_mfma(const rq_qweight &w, const void *x, void *y, rq_dtype yt, int m, hipStream_t s) {
    return launch_mfma(w, nullptr, x, y, yt, m, s);
}

int launch_swiglu_mfma(const rq_qweight &gate, const rq_qweight &up, const void *x, void *h, int m, hipStream_t s) {
    return launch_mfma(gate, &up, x, h, RQ_F16, m, s);
}

}  // namespace rq
