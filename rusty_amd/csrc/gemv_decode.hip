// Decode dequant-GEMV, m <= 4:  Y[m, n] = sum_k X[m, k] * deq(W)[n, k], fp16
// activations (f32 ones, m <= 2, carried as two fp16 terms each: see XF).
// Serves m = 1-2, and m = 3-4 for the weights the MFMA GEMV does not take
// (affine codes); per-row codes at m >= 3 go to the MFMA GEMV.
//
// HBM-bound: every weight byte is read once, 16.8 MB for a 4096x4096 layer,
// a few microseconds per call.  At that size the fixed costs of a launch (wave
// dispatch, first-byte latency, the reduction tail) are a large part of the
// time, so the kernel is shaped around them (measured on MI355X, one-shot
// 16 MB reads: ~3.8-4.1 us floor):
//  * One block of 256 threads owns R*RP rows.  Thread tt of a row group (TPR
//    threads) owns the 16-byte chunks tt, tt+TPR, ... of each of its rows, so
//    every wave-wide load is 1 KiB contiguous in one row -- the access
//    pattern that streams best (row-interleaved patterns measured 1.3-3x
//    slower).  Many small blocks spread the dispatch over all 256 CUs.
//  * Loads are buffer loads: the X slice first (cached), then all R*CPT weight
//    chunks with the non-temporal policy (the weights are read once).  Rows
//    past N and chunks past K are offsets past the buffer resource, which the
//    hardware returns as zeros: no branches around the loads.
//  * int8 -> fp16 is exact and convert-free: XOR 0x80 gives q+128, v_perm_b32
//    puts it under exponent 0x64 -> fp16 1152+q; v_dot2_f32_f16 multiplies
//    with X in f32; the lane subtracts 1152 * (sum of its X slice) once.
//    Affine (reference) codes skip the XOR: fp16 1024+u, and per chunk the
//    lane applies its group's scale s and bias b:
//    acc += s * sum (1024+u) x + (b - 1024 s) * sum x.
//  * Reduction: every thread stores its R*M partials to LDS; after one
//    barrier each wave owns whole (row, token) tasks: TPR partials are summed
//    with LDS reads + four DPP row steps + four readlanes, with no LDS
//    round trip per row and no cross-lane shuffles.
#include "common.hpp"

namespace rq {
namespace {

constexpr int DT = 256;
constexpr uint32_t kOOB = 0x80000000u;  // any offset past a resource reads zero
// output modes: f32 store, fp16 store, f32 accumulate (y += result)
constexpr int kYF32 = 0, kYF16 = 1, kYAdd = 2;

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), 0, bytes, 0x00020000);
}
// aux bit 1 = non-temporal (streamed once), 0 = default caching
template <int AUX>
__device__ __forceinline__ uint4 bload(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const u32x4 v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, AUX));
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2_t, a), __builtin_bit_cast(h2_t, b), c, false);
}
__device__ __forceinline__ uint32_t magic_lo(uint32_t w) { return __builtin_amdgcn_perm(0x64646464u, w, 0x04010400u); }
__device__ __forceinline__ uint32_t magic_hi(uint32_t w) { return __builtin_amdgcn_perm(0x64646464u, w, 0x04030402u); }

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float readlane(float v, int l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}
// Sum over the 64 lanes, result uniform (scalar) across the wave.
__device__ __forceinline__ float wave_total(float v) {
    v += dpp<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp<0x141>(v);  // row_half_mirror
    v += dpp<0x140>(v);  // row_mirror: each 16-lane row holds its sum
    return (readlane(v, 0) + readlane(v, 16)) + (readlane(v, 32) + readlane(v, 48));
}

__device__ __forceinline__ float silu(float v) { return v / (1.0f + expf(-v)); }

// M: activation rows (m_act <= M); CPT: chunks per thread; TPR: threads per
// row group; R: rows per row group; FMT: 0 = ROWWISE_I8, 1 = AFFINE_U8.
// SWI: SwiGLU gate/up pass -- W/scales/biases are the gate weight,
// W2/scales2/biases2 the up weight of the same shape and format; the block
// loads R gate rows and the same R up rows per row group and writes
// h = silu(g) * u (fp16).
// NORM (m = 1): the activation row is RMSNorm(x) computed in the prologue
// from the f32 row Xf and the fp16 norm weight NW (kernels.wgsl:87-102):
// xn = fp16((x * inv) * nw), inv = 1 / sqrt(mean(x^2) + eps).  Each block
// reduces the sum of squares itself (one barrier) after its weight loads are
// in flight, so the norm costs no launch and hides under the weight stream.
// SA > 0 (m = 1): the activation row is decode attention's output, combined
// in the prologue from SA partial softmaxes per head (the attention kernel's
// split over positions): Xf holds o[head][SA][attn_hd] (fp16, each split's
// output normalised by its own sum) followed by (m, l)[head][SA] (float2);
// x = sum_s w_s o_s / sum_s w_s, w_s = e^(m_s - M) l_s, M = max_s m_s, rounded
// to fp16 and shared through LDS like the norm's row.
// ROPE (with NORM, m = 1): the weight is a Llama layer's packed [q; k; v]
// (rd.hd rows per head) and the block's local rows come in rotate-half pairs:
// local rows 2p and 2p + 1 are rows d and d + hd/2 of one head, global pair
// P = block * ROWS/2 + p covering head P / (hd/2), d = P % (hd/2).  A wave
// reduces both rows of a pair, so the epilogue rotates them in registers --
// a = y[d], b = y[d + hd/2]: o[d] = a cos - b sin, o[d + hd/2] = a sin +
// b cos, angle pos * theta^(-2d/hd) from the table at the step's position
// (kernels.wgsl:60-79) -- and writes q (f32) to rd.q, k (rotated) and v
// (fp16) into the caches at that position (rusty-graph/src/lib.rs:235-246).
// XF (no NORM / SA): the activations are f32 (Xf).  Each 16-value chunk of a
// row is scaled by a power of two 2^-e that puts its largest magnitude in
// [2^14, 2^15) (exact), every scaled value is split into two fp16 terms
// hi = fp16(v), lo = fp16(v - hi) (their sum equals v to ~2^-22 relative),
// and the chunk's partial sums are multiplied back by 2^e: any finite f32
// row is carried without overflowing fp16, and small values keep f32
// accuracy instead of fp16's subnormal spacing.
template <int M, int CPT, int TPR, int R, int FMT, bool SWI, bool NORM, int SA = 0, bool XF = false, bool ROPE = false>
__global__ __launch_bounds__(DT) void k_gemv_decode(const uint8_t *__restrict__ W, const float *__restrict__ scales,
                                                    const float *__restrict__ biases,
                                                    const uint8_t *__restrict__ W2, const float *__restrict__ scales2,
                                                    const float *__restrict__ biases2,
                                                    const _Float16 *__restrict__ X, const float *__restrict__ Xf,
                                                    const _Float16 *__restrict__ NW, float eps,
                                                    void *__restrict__ Yv, int ymode, int m_act, int N, int K,
                                                    int group, int attn_hd, RopeDecode rd) {
    static_assert(!NORM || M == 1, "the fused norm serves one activation row");
    static_assert(SA == 0 || (M == 1 && !NORM && !SWI), "the attention combine serves one activation row");
    static_assert(!XF || (!NORM && SA == 0), "f32 activations replace the plain fp16 row");
    static_assert(!ROPE || (NORM && !SWI), "the rotary epilogue serves the normed q/k/v projection");
    constexpr int RP = DT / TPR;
    constexpr int ROWS = R * RP;
    constexpr int TASKS = ROWS * M;
    constexpr int NR = SWI ? 2 * R : R;  // weight rows loaded per row group
    static_assert(!ROPE || ROWS % 2 == 0, "rotary pairs: an even number of rows per block");
    constexpr int PAIRS = ROWS / 2;
    __shared__ float part[SWI ? 2 * TASKS : TASKS][TPR];

    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int rp = t / TPR, tt = t % TPR;
    const int C = K >> 4;
    const int row0 = blockIdx.x * ROWS;
    // ROPE: the step's position, requested first (the epilogue's table reads
    // and cache writes depend on it); rotary pairs of this block
    const int pos = ROPE ? *rd.pos : 0;
    const int half = ROPE ? rd.hd / 2 : 1;
    const int pairs_here = ROPE ? min(PAIRS, N / 2 - (int)blockIdx.x * PAIRS) : 0;
    // ROPE: head and d of the block's first pair (one division per block,
    // uniform); a block's pairs (PAIRS < hd/2) cross at most one head boundary
    const int p_first = ROPE ? (int)blockIdx.x * PAIRS : 0;
    const int head0 = ROPE ? p_first / half : 0, d0 = ROPE ? p_first - head0 * half : 0;
    // the weight row of local row lr (ROPE: pair lr / 2, row d or d + hd/2 of its head)
    auto wrow = [&](int lr) -> int {
        if constexpr (ROPE) {
            const int dd = d0 + lr / 2, wrap = dd >= half ? 1 : 0;
            return (head0 + wrap) * rd.hd + (dd - wrap * half) + (lr & 1) * half;
        } else {
            return row0 + lr;
        }
    };

    // X slice (issued first so its wait does not cover the weight stream).
    // NORM: the block loads the f32 row and the norm weight once, spread over
    // all its threads (chunk c by thread c % DT), and shares the normalised
    // fp16 row through LDS -- not once per row group.
    constexpr int XC = CPT * TPR;            // chunks the row groups cover
    constexpr int NL = (XC + DT - 1) / DT;   // NORM: chunks loaded per thread
    uint32_t xh[CPT][M][8];
    // XF: x = 2^e (xh + xl) to ~2^-22 relative, pe = 2^e per chunk and row
    uint32_t xl[XF ? CPT : 1][XF ? M : 1][8];
    float pe[XF ? CPT : 1][XF ? M : 1];
    uint4 xf4[NORM ? NL : 1][4], nw4[NORM ? NL : 1][2];
    // SA: 8-element pieces of the row, piece u by thread u % DT: SA (m, l)
    // pairs of its head and SA x 8 fp16 partial outputs
    constexpr int NU = (2 * XC + DT - 1) / DT;
    constexpr int SAL = SA > 0 ? SA : 1;
    uint4 pacc[SA > 0 ? NU : 1][SAL][1], pml[SA > 0 ? NU : 1][(SAL + 1) / 2];
    if constexpr (SA > 0) {
        const int nh = K / attn_hd;
        const auto racc = make_rsrc(Xf, (uint32_t)nh * SA * (uint32_t)attn_hd * 2u);
        const auto rml = make_rsrc(Xf + (size_t)nh * SA * attn_hd / 2, (uint32_t)nh * SA * 8u);
#pragma unroll
        for (int j = 0; j < NU; ++j) {
            const int u = t + DT * j;
            const bool live = u < 2 * C;
            const int e0 = u * 8, h = e0 / attn_hd, d0 = e0 - h * attn_hd;
#pragma unroll
            for (int q = 0; q < (SAL + 1) / 2; ++q)
                pml[j][q] = bload<0>(rml, live ? (uint32_t)(h * SA + 2 * q) * 8u : kOOB);
#pragma unroll
            for (int sp = 0; sp < SAL; ++sp) {
                const uint32_t off = live ? ((uint32_t)(h * SA + sp) * attn_hd + d0) * 2u : kOOB;
                pacc[j][sp][0] = bload<0>(racc, off);
            }
        }
    } else if constexpr (NORM) {
        const auto rxf = make_rsrc(Xf, (uint32_t)K * 4u);
        const auto rnw = make_rsrc(NW, (uint32_t)K * 2u);
#pragma unroll
        for (int j = 0; j < NL; ++j) {
            const int c = t + DT * j;
            const uint32_t off = c < C ? (uint32_t)c * 64u : kOOB, offw = c < C ? (uint32_t)c * 32u : kOOB;
#pragma unroll
            for (int q = 0; q < 4; ++q) xf4[j][q] = bload<0>(rxf, off + 16 * q);
            nw4[j][0] = bload<0>(rnw, offw);
            nw4[j][1] = bload<0>(rnw, offw + 16);
        }
    } else if constexpr (XF) {
        // f32 activations (the reference's dtype): 64 bytes per chunk, each
        // value split into two fp16 terms in registers
        const auto rx = make_rsrc(Xf, (uint32_t)m_act * (uint32_t)K * 4u);
#pragma unroll
        for (int j = 0; j < CPT; ++j) {
            const int c = tt + TPR * j;
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const uint32_t off = c < C ? ((uint32_t)m * K + (uint32_t)c * 16) * 4u : kOOB;
                uint4 f4[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) f4[q] = bload<0>(rx, off + 16 * q);
                float amax = 0.0f;
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    amax = fmaxf(fmaxf(fmaxf(amax, fabsf(__builtin_bit_cast(float, f4[q].x))),
                                       fmaxf(fabsf(__builtin_bit_cast(float, f4[q].y)),
                                             fabsf(__builtin_bit_cast(float, f4[q].z)))),
                                 fabsf(__builtin_bit_cast(float, f4[q].w)));
                // amax = f * 2^E, f in [0.5, 1): 2^-(E - 15) maps it into [2^14, 2^15)
                // (a zero, infinite or NaN maximum gives E = 0: the values pass
                // through scaled by 2^15 and an inf or NaN stays one)
                const int ex = max(__builtin_amdgcn_frexp_expf(amax) - 15, -126);
                pe[j][m] = __builtin_amdgcn_ldexpf(1.0f, ex);
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float f[4] = {__builtin_amdgcn_ldexpf(__builtin_bit_cast(float, f4[q].x), -ex),
                                        __builtin_amdgcn_ldexpf(__builtin_bit_cast(float, f4[q].y), -ex),
                                        __builtin_amdgcn_ldexpf(__builtin_bit_cast(float, f4[q].z), -ex),
                                        __builtin_amdgcn_ldexpf(__builtin_bit_cast(float, f4[q].w), -ex)};
#pragma unroll
                    for (int e = 0; e < 2; ++e) {
                        const h2_t h = {(_Float16)f[2 * e], (_Float16)f[2 * e + 1]};
                        const h2_t l = {(_Float16)(f[2 * e] - (float)h.x), (_Float16)(f[2 * e + 1] - (float)h.y)};
                        xh[j][m][2 * q + e] = __builtin_bit_cast(uint32_t, h);
                        xl[j][m][2 * q + e] = __builtin_bit_cast(uint32_t, l);
                    }
                }
            }
        }
    } else {
        const auto rx = make_rsrc(X, (uint32_t)m_act * (uint32_t)K * 2u);
#pragma unroll
        for (int j = 0; j < CPT; ++j) {
            const int c = tt + TPR * j;
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const uint32_t off = c < C ? ((uint32_t)m * K + (uint32_t)c * 16) * 2u : kOOB;
                const uint4 a = bload<0>(rx, off), b = bload<0>(rx, off + 16);
                xh[j][m][0] = a.x; xh[j][m][1] = a.y; xh[j][m][2] = a.z; xh[j][m][3] = a.w;
                xh[j][m][4] = b.x; xh[j][m][5] = b.y; xh[j][m][6] = b.z; xh[j][m][7] = b.w;
            }
        }
    }
    const int rows_here = ROPE ? 2 * pairs_here : min(ROWS, N - row0);  // ROPE: local rows 0 .. 2 pairs_here
    // Per-row scales of the tasks this wave will finish, requested before the
    // weights (and above the prologue's barriers, which the compiler does not
    // move loads across) so the epilogue does not wait on a global load after
    // the reduction; issued after the weights, they made the prologue's waits
    // for its activation row count the weight loads too.
    constexpr int NTW = (TASKS + DT / 64 - 1) / (DT / 64);  // tasks per wave
    float srow[NTW], srow2[SWI ? NTW : 1];
    if constexpr (FMT == 0 && !ROPE) {
#pragma unroll
        for (int i = 0; i < NTW; ++i) {
            const int rin = (wave + (DT / 64) * i) / M;
            const bool ok = wave + (DT / 64) * i < TASKS && rin < rows_here;
            srow[i] = ok ? scales[row0 + rin] : 0.0f;
            if constexpr (SWI) srow2[i] = ok ? scales2[row0 + rin] : 0.0f;
        }
    }
    // ROPE: wave w finishes pairs w, w + 4, ...: their rows' scales (here)
    // and the (cos, sin) of their d at the position (after the weight loads:
    // they wait for the position, which must not hold back the weight stream)
    constexpr int NPW = (PAIRS + DT / 64 - 1) / (DT / 64);
    float rs0[ROPE ? NPW : 1], rs1[ROPE ? NPW : 1];
    float2 rcs[ROPE ? NPW : 1];
    if constexpr (ROPE) {
#pragma unroll
        for (int i = 0; i < NPW; ++i) {
            // branch-free: an index past the block's pairs reads row 0's scale, zeroed
            const int pr = wave + (DT / 64) * i;
            const bool ok = pr < pairs_here;
            if constexpr (FMT == 0) {
                const float a = scales[ok ? wrow(2 * pr) : 0], b = scales[ok ? wrow(2 * pr + 1) : 0];
                rs0[i] = ok ? a : 0.0f;
                rs1[i] = ok ? b : 0.0f;
            }
        }
    }
    // y += result: the old values of the residual, requested now for the same reason
    float yold[NTW];
#pragma unroll
    for (int i = 0; i < NTW; ++i) {
        const int task = wave + (DT / 64) * i, rin = task / M, m = task % M;
        yold[i] = (!ROPE && ymode == kYAdd && task < TASKS && rin < rows_here && m < m_act)
                      ? reinterpret_cast<const float *>(Yv)[(size_t)m * N + row0 + rin]
                      : 0.0f;
    }
    // Affine: the group scale and bias of every chunk (group % 16 == 0 and
    // K % group == 0, so a chunk sits in one group: row * (K / group) + c * 16 / group).
    float sg[NR][CPT], bg[NR][CPT];
    if constexpr (FMT == 1) {
        const int gk = K / group;
        int cg[CPT];
#pragma unroll
        for (int j = 0; j < CPT; ++j) cg[j] = (int)((unsigned)(tt + TPR * j) * 16u / (unsigned)group);
#pragma unroll
        for (int r = 0; r < NR; ++r) {
            const float *sp = r < R ? scales : scales2, *bp = r < R ? biases : biases2;
            const int rin = (r % R) * RP + rp;
#pragma unroll
            for (int j = 0; j < CPT; ++j) {
                // branch-free (a branch around each load made every one wait
                // for the previous): a chunk past K multiplies zero activations
                // and a row past N is not stored, so those take group 0's values
                const int c = tt + TPR * j;
                const size_t g = c < C && rin < rows_here ? (size_t)wrow(rin) * gk + cg[j] : 0;
                sg[r][j] = sp[g];
                bg[r][j] = bp ? bp[g] : 0.0f;
            }
        }
    }

    // Weight chunks: R rows x CPT chunks per thread, all in flight.  ROPE:
    // one resource over the whole weight, rows by the pair mapping.
    const auto rw = ROPE ? make_rsrc(W, (uint32_t)N * (uint32_t)K)
                         : make_rsrc(W + (size_t)row0 * K, (uint32_t)rows_here * (uint32_t)K);
    const auto rw2 = make_rsrc((SWI ? W2 : W) + (size_t)row0 * K, (uint32_t)rows_here * (uint32_t)K);
    uint4 w[NR][CPT];
#pragma unroll
    for (int r = 0; r < NR; ++r)
#pragma unroll
        for (int j = 0; j < CPT; ++j) {
            const int c = tt + TPR * j, lr = (r % R) * RP + rp;
            uint32_t off = c < C ? (uint32_t)lr * (uint32_t)K + (uint32_t)c * 16 : kOOB;
            if constexpr (ROPE) off = c < C && lr < rows_here ? (uint32_t)wrow(lr) * (uint32_t)K + (uint32_t)c * 16 : kOOB;
            w[r][j] = bload<2>(r < R ? rw : rw2, off);
        }
    if constexpr (ROPE) {
#pragma unroll
        for (int i = 0; i < NPW; ++i) {
            const int pr = wave + (DT / 64) * i;
            const int dd = d0 + pr, d = dd >= half ? dd - half : dd;
            rcs[i] = rd.rope[(size_t)pos * half + (pr < pairs_here ? d : 0)];
        }
    }
    if constexpr (SA > 0) {
        __shared__ uint4 xsa[XC * 2];  // the combined fp16 row, 2 x 16 B per chunk
#pragma unroll
        for (int j = 0; j < NU; ++j) {
            const int u = t + DT * j;
            if (u >= 2 * XC) break;
            float mv[SAL], lv[SAL];
#pragma unroll
            for (int sp = 0; sp < SAL; ++sp) {
                const uint4 v = pml[j][sp / 2];
                mv[sp] = __builtin_bit_cast(float, (sp & 1) ? v.z : v.x);
                lv[sp] = __builtin_bit_cast(float, (sp & 1) ? v.w : v.y);
            }
            float mx = mv[0];
#pragma unroll
            for (int sp = 1; sp < SAL; ++sp) mx = fmaxf(mx, mv[sp]);
            float wgt[SAL], den = 0.0f;
#pragma unroll
            for (int sp = 0; sp < SAL; ++sp) {
                wgt[sp] = expf(mv[sp] - mx) * lv[sp];  // an empty split's m = -inf weighs 0
                den += wgt[sp];
            }
            const float inv = 1.0f / den;
            float o[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] = 0.0f;
#pragma unroll
            for (int sp = 0; sp < SAL; ++sp) {
                const uint4 a = pacc[j][sp][0];
                const uint32_t wd[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const h2_t hv = __builtin_bit_cast(h2_t, wd[e]);
                    o[2 * e] = __builtin_fmaf(wgt[sp], (float)hv.x, o[2 * e]);
                    o[2 * e + 1] = __builtin_fmaf(wgt[sp], (float)hv.y, o[2 * e + 1]);
                }
            }
            uint32_t hv[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const h2_t pr = {(_Float16)(o[2 * q] * inv), (_Float16)(o[2 * q + 1] * inv)};
                hv[q] = __builtin_bit_cast(uint32_t, pr);
            }
            // pieces past the row (chunks the row groups cover beyond K) hold zeros
            xsa[u] = u < 2 * C ? make_uint4(hv[0], hv[1], hv[2], hv[3]) : make_uint4(0, 0, 0, 0);
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < CPT; ++j) {
            const int c = tt + TPR * j;
            const uint4 a = xsa[2 * c], b = xsa[2 * c + 1];
            xh[j][0][0] = a.x; xh[j][0][1] = a.y; xh[j][0][2] = a.z; xh[j][0][3] = a.w;
            xh[j][0][4] = b.x; xh[j][0][5] = b.y; xh[j][0][6] = b.z; xh[j][0][7] = b.w;
        }
    }
    if constexpr (NORM) {
        // sum of squares of the row (chunks past K loaded as zero), one barrier
        __shared__ float nred[DT / 64];
        __shared__ uint4 xsh[XC * 2];  // the normalised fp16 row, 2 x 16 B per chunk
        float ss = 0.0f;
#pragma unroll
        for (int j = 0; j < NL; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float f[4] = {__builtin_bit_cast(float, xf4[j][q].x), __builtin_bit_cast(float, xf4[j][q].y),
                                    __builtin_bit_cast(float, xf4[j][q].z), __builtin_bit_cast(float, xf4[j][q].w)};
#pragma unroll
                for (int e = 0; e < 4; ++e) ss = __builtin_fmaf(f[e], f[e], ss);
            }
        ss = wave_total(ss);
        if (lane == 0) nred[wave] = ss;
        __syncthreads();
        ss = (nred[0] + nred[1]) + (nred[2] + nred[3]);
        const float inv = 1.0f / sqrtf(ss / (float)K + eps);
#pragma unroll
        for (int j = 0; j < NL; ++j) {
            const int c = t + DT * j;
            if (c >= XC) break;
            uint32_t hv[8];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint4 xv = xf4[j][q];
                const float f[4] = {__builtin_bit_cast(float, xv.x), __builtin_bit_cast(float, xv.y),
                                    __builtin_bit_cast(float, xv.z), __builtin_bit_cast(float, xv.w)};
                // norm weights of elements 4q..4q+3: halves 4q..4q+3 of the chunk's 16
                const uint4 nv = nw4[j][q >> 1];
                const uint32_t n01 = (q & 1) ? nv.z : nv.x, n23 = (q & 1) ? nv.w : nv.y;
                const h2_t a = __builtin_bit_cast(h2_t, n01), b = __builtin_bit_cast(h2_t, n23);
                const h2_t lo = {(_Float16)((f[0] * inv) * (float)a.x), (_Float16)((f[1] * inv) * (float)a.y)};
                const h2_t hi = {(_Float16)((f[2] * inv) * (float)b.x), (_Float16)((f[3] * inv) * (float)b.y)};
                hv[2 * q] = __builtin_bit_cast(uint32_t, lo);
                hv[2 * q + 1] = __builtin_bit_cast(uint32_t, hi);
            }
            xsh[2 * c] = make_uint4(hv[0], hv[1], hv[2], hv[3]);
            xsh[2 * c + 1] = make_uint4(hv[4], hv[5], hv[6], hv[7]);
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < CPT; ++j) {
            const int c = tt + TPR * j;
            const uint4 a = xsh[2 * c], b = xsh[2 * c + 1];
            xh[j][0][0] = a.x; xh[j][0][1] = a.y; xh[j][0][2] = a.z; xh[j][0][3] = a.w;
            xh[j][0][4] = b.x; xh[j][0][5] = b.y; xh[j][0][6] = b.z; xh[j][0][7] = b.w;
        }
    }
    // Per-chunk sums of X (fp16 dot with (1,1)); zero for chunks past K.
    float xs[CPT][M], xs_tot[M];
#pragma unroll
    for (int m = 0; m < M; ++m) xs_tot[m] = 0.0f;
#pragma unroll
    for (int j = 0; j < CPT; ++j)
#pragma unroll
        for (int m = 0; m < M; ++m) {
            float s = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; ++i) s = dot2(xh[j][m][i], 0x3C003C00u, s);
            if constexpr (XF) {
#pragma unroll
                for (int i = 0; i < 8; ++i) s = dot2(xl[j][m][i], 0x3C003C00u, s);
                s *= pe[j][m];
            }
            xs[j][m] = s;
            xs_tot[m] += s;
        }

#pragma unroll
    for (int r = 0; r < NR; ++r) {
        float p[M];
#pragma unroll
        for (int m = 0; m < M; ++m) p[m] = 0.0f;
#pragma unroll
        for (int j = 0; j < CPT; ++j) {
            const uint32_t wd[4] = {w[r][j].x, w[r][j].y, w[r][j].z, w[r][j].w};
            float d[M];
#pragma unroll
            for (int m = 0; m < M; ++m) d[m] = FMT == 0 && !XF ? p[m] : 0.0f;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint32_t u = FMT == 0 ? (wd[q] ^ 0x80808080u) : wd[q];
                uint32_t lo = magic_lo(u), hi = magic_hi(u);
                if constexpr (XF) {
                    // exact code values (q, or u for affine) rather than the
                    // offset ones: at f32 accuracy the offset's products would
                    // cancel against the correction term
                    const h2_t off = FMT == 0 ? (h2_t){(_Float16)1152.0f, (_Float16)1152.0f}
                                              : (h2_t){(_Float16)1024.0f, (_Float16)1024.0f};
                    lo = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2_t, lo) - off);
                    hi = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2_t, hi) - off);
                }
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    d[m] = dot2(lo, xh[j][m][2 * q], d[m]);
                    d[m] = dot2(hi, xh[j][m][2 * q + 1], d[m]);
                    if constexpr (XF) {
                        d[m] = dot2(lo, xl[j][m][2 * q], d[m]);
                        d[m] = dot2(hi, xl[j][m][2 * q + 1], d[m]);
                    }
                }
            }
#pragma unroll
            for (int m = 0; m < M; ++m) {
                // XF: the chunk's sums are in units of 2^-e; pe = 2^e restores them
                if constexpr (FMT == 0) {
                    p[m] = XF ? __builtin_fmaf(pe[j][m], d[m], p[m]) : d[m];
                } else {
                    const float s = sg[r][j];
                    const float c = XF ? bg[r][j] : __builtin_fmaf(-1024.0f, s, bg[r][j]);
                    p[m] = __builtin_fmaf(s, XF ? d[m] * pe[j][m] : d[m], p[m]);
                    p[m] = __builtin_fmaf(c, xs[j][m], p[m]);
                }
            }
        }
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const float v = FMT == 0 && !XF ? __builtin_fmaf(-1152.0f, xs_tot[m], p[m]) : p[m];
            // up rows (r >= R) land TASKS entries after their gate rows
            part[(r / R) * TASKS + ((r % R) * RP + rp) * M + m][tt] = v;
        }
    }
    __syncthreads();

    if constexpr (ROPE) {
        // Each wave finishes whole rotary pairs: both rows' sums, the rotation,
        // the stores (q f32; k and v fp16 into the caches at the position).
#pragma unroll
        for (int i = 0; i < NPW; ++i) {
            const int pr = wave + (DT / 64) * i;
            if (pr >= PAIRS) break;
            float v0 = 0.0f, v1 = 0.0f;
#pragma unroll
            for (int u = 0; u < TPR / 64; ++u) {
                v0 += part[2 * pr][lane + 64 * u];
                v1 += part[2 * pr + 1][lane + 64 * u];
            }
            const float a0 = wave_total(v0), a1 = wave_total(v1);
            if (lane == 0 && pr < pairs_here) {
                const float y0 = FMT == 0 ? a0 * rs0[i] : a0, y1 = FMT == 0 ? a1 * rs1[i] : a1;
                const int dd = d0 + pr, wrap = dd >= half ? 1 : 0;
                const int head = head0 + wrap, d = dd - wrap * half;
                const float c = rcs[i].x, sn = rcs[i].y;
                if (head < rd.n_heads) {
                    float *qh = rd.q + (size_t)head * rd.hd;
                    qh[d] = y0 * c - y1 * sn;
                    qh[d + half] = y0 * sn + y1 * c;
                } else if (head < rd.n_heads + rd.n_kv) {
                    _Float16 *kh = rd.kc + ((size_t)(head - rd.n_heads) * rd.max_seq + pos) * rd.hd;
                    kh[d] = (_Float16)(y0 * c - y1 * sn);
                    kh[d + half] = (_Float16)(y0 * sn + y1 * c);
                } else {
                    _Float16 *vh = rd.vc + ((size_t)(head - rd.n_heads - rd.n_kv) * rd.max_seq + pos) * rd.hd;
                    vh[d] = (_Float16)y0;
                    vh[d + half] = (_Float16)y1;
                }
            }
        }
        return;
    }

    // Each wave finishes whole (row, token) tasks.
#pragma unroll
    for (int i_t = 0; i_t < NTW; ++i_t) {
        const int task = wave + (DT / 64) * i_t;
        if (task >= TASKS) break;
        float v = 0.0f, v2 = 0.0f;
#pragma unroll
        for (int i = 0; i < TPR / 64; ++i) v += part[task][lane + 64 * i];
        if constexpr (SWI) {
#pragma unroll
            for (int i = 0; i < TPR / 64; ++i) v2 += part[TASKS + task][lane + 64 * i];
        }
        const float tot = wave_total(v);
        const float tot2 = SWI ? wave_total(v2) : 0.0f;
        const int rin = task / M, m = task % M;
        const int row = row0 + rin;
        if (lane == 0 && rin < rows_here && m < m_act) {
            float y = FMT == 0 ? tot * srow[i_t] : tot;
            if constexpr (SWI) y = silu(y) * (FMT == 0 ? tot2 * srow2[i_t] : tot2);
            const size_t o = (size_t)m * N + row;
            if (ymode == kYF16) reinterpret_cast<_Float16 *>(Yv)[o] = (_Float16)y;
            else if (ymode == kYAdd) reinterpret_cast<float *>(Yv)[o] = yold[i_t] + y;
            else reinterpret_cast<float *>(Yv)[o] = y;
        }
    }
}

using DecodeFn = void (*)(const uint8_t *, const float *, const float *, const uint8_t *, const float *,
                          const float *, const _Float16 *, const float *, const _Float16 *, float, void *, int, int, int, int, int,
                          int, RopeDecode);

// A kernel instance and the rows per row group (R) it was compiled for; the
// grid is derived from the same R.
struct Decode {
    DecodeFn fn;
    int r;
};
template <int M, int CPT, int TPR, int R, int FMT, bool SWI, bool NORM, int SA = 0, bool XF = false, bool ROPE = false>
constexpr Decode inst() { return {&k_gemv_decode<M, CPT, TPR, R, FMT, SWI, NORM, SA, XF, ROPE>, R}; }

// Rows per row group, measured on MI355X with the weights streamed from HBM:
//  m = 1:
//   * SwiGLU pass (R gate + R up rows): 2 pairs; 4 with the fused norm at
//     row groups of <= 128 threads (gate/up 5632x2048: 6.90 -> 6.69 us;
//     11008x4096 without norm, 1 -> 2 pairs: 15.4 -> 14.7 us);
//   * tall weights (n_out >= 16384, e.g. an lm_head): 8 -- fewer blocks, each
//     re-reading the activation row less per weight byte (32000x2048 + norm:
//     15.7 -> 13.0 us);
//   * fused norm at row groups of <= 128 threads: 6 -- the f32 row and the
//     norm weight (6 B per element) are read by every block, so more rows per
//     block (qkv 3072x2048 + norm: 3.98 -> 3.59 us);
//   * two or more chunks per thread (k_in > 4096): 4 (2048x5632: 4.26 -> 4.17 us);
//     affine codes keep 2 (4 measured 4096x4096 5.19 -> 5.14 us, but the 1.1B
//     decode step's down projection, 2048x5632, 1886 -> 1860 tok/s);
//   * f32 activations, row groups of 256 threads: every block reads the whole
//     f32 row (4 B per element, twice the fp16 row), so 8 rows while that
//     leaves >= 1024 blocks (>= 512 past k_in = 4096), else 4 while >= 1024,
//     else 2 (us for 2 / 4 / 8 rows: 4096x4096 5.76 / 5.23 / 5.56, affine
//     6.18 / 5.60 / 5.60, 11008x4096 11.1 / 10.15 / 10.05, 4096x11008 - /
//     11.55 / 10.6, 2048x2048 3.25 / 3.40 / 3.90);
//   * otherwise 2.
//  m = 2..4: 4 (SwiGLU: 2 pairs, 4 at m = 2 and 256 threads); 8 for f32 activations at m = 2 while that
//  leaves >= 512 blocks (4096x4096 6.94 -> 6.40 us; fp16 stays at 4: 5.30 vs 5.62).
//   * attention-combine prologue: 4 (each block re-reads the partials, so
//     fewer, larger blocks).
// fmt: 0 = per-row int8, 1 = affine u8; swi selects the SwiGLU gate/up
// pass; norm (m = 1) the fused RMSNorm prologue; sa (m = 1) the attention
// combine of sa partials per head; xf (m <= 2, no norm / sa) f32 activations:
// 0 for fp16, else the rows per block for f32 rows (m = 1: 2, 4 or 8; m = 2: 4 or 8).
template <int M, int CPT, int TPR, int FMT>
Decode pick_fmt(bool swi, bool norm, bool tall, int sa, int xf, bool rope) {
    if constexpr (M == 1) {
        constexpr int RN = TPR <= 128 ? 6 : 2;   // fused norm
        constexpr int RSN = TPR <= 128 ? 4 : 2;  // SwiGLU pairs with the fused norm
        constexpr int RP = FMT == 0 && CPT >= 2 ? 4 : 2;
        if (rope) return inst<1, CPT, TPR, RN, FMT, false, true, 0, false, true>();
        if (sa == 1) return inst<1, CPT, TPR, 4, FMT, false, false, 1>();
        if (sa == 2) return inst<1, CPT, TPR, 4, FMT, false, false, 2>();
        if (sa == 4) return inst<1, CPT, TPR, 4, FMT, false, false, 4>();
        if (sa == 8) return inst<1, CPT, TPR, 4, FMT, false, false, 8>();
        if (swi) {
            if (norm) return inst<1, CPT, TPR, RSN, FMT, true, true>();
            // f32 row at 256-thread row groups: 4 pairs (11008x4096 MLP 25.5 -> 24.7 us;
            // the fp16 row keeps 2: 23.3 either way)
            if (xf) return inst<1, CPT, TPR, TPR == 256 ? 4 : 2, FMT, true, false, 0, true>();
            return inst<1, CPT, TPR, 2, FMT, true, false>();
        }
        if (FMT == 0 && tall) {
            if (norm) return inst<1, CPT, TPR, 8, FMT, false, true>();
            return xf ? inst<1, CPT, TPR, 8, FMT, false, false, 0, true>() : inst<1, CPT, TPR, 8, FMT, false, false>();
        }
        if (norm) return inst<1, CPT, TPR, RN, FMT, false, true>();
        if (xf) {
            // f32 row: xf rows per block where the row group is the whole block
            if constexpr (TPR == 256) {
                if (xf == 8) return inst<1, CPT, TPR, 8, FMT, false, false, 0, true>();
                if (xf == 4) return inst<1, CPT, TPR, 4, FMT, false, false, 0, true>();
                return inst<1, CPT, TPR, 2, FMT, false, false, 0, true>();
            }
            return inst<1, CPT, TPR, RP, FMT, false, false, 0, true>();
        }
        return inst<1, CPT, TPR, RP, FMT, false, false>();
    } else if constexpr (M == 2) {
        (void)norm;
        (void)tall;
        (void)sa;
        (void)rope;
        // SwiGLU at 256-thread row groups: 4 pairs (11008x4096 MLP, m = 2: fp16
        // 26.45 -> 25.95 us, f32 activations 34.35 -> 30.1)
        constexpr int RS2 = TPR == 256 ? 4 : 2;
        if (swi) return xf ? inst<2, CPT, TPR, RS2, FMT, true, false, 0, true>() : inst<2, CPT, TPR, RS2, FMT, true, false>();
        if (xf == 8) return inst<2, CPT, TPR, 8, FMT, false, false, 0, true>();
        return xf ? inst<2, CPT, TPR, 4, FMT, false, false, 0, true>() : inst<2, CPT, TPR, 4, FMT, false, false>();
    } else {
        (void)norm;
        (void)tall;
        (void)sa;
        (void)xf;
        (void)rope;
        if (swi) return inst<M, CPT, TPR, 2, FMT, true, false>();
        return inst<M, CPT, TPR, 4, FMT, false, false>();
    }
}

template <int M, int CPT, int TPR>
Decode pick_swi(int fmt, bool swi, bool norm, bool tall, int sa, int xf, bool rope) {
    return fmt == 0 ? pick_fmt<M, CPT, TPR, 0>(swi, norm, tall, sa, xf, rope)
                    : pick_fmt<M, CPT, TPR, 1>(swi, norm, tall, sa, xf, rope);
}

template <int M, int CPT>
Decode pick_tpr(int tpr, int fmt, bool swi, bool norm, bool tall, int sa, int xf, bool rope) {
    switch (tpr) {
    case 64: return pick_swi<M, CPT, 64>(fmt, swi, norm, tall, sa, xf, rope);
    case 128: return pick_swi<M, CPT, 128>(fmt, swi, norm, tall, sa, xf, rope);
    default: return pick_swi<M, CPT, 256>(fmt, swi, norm, tall, sa, xf, rope);
    }
}

template <int M>
Decode pick_cpt(int cpt, int tpr, int fmt, bool swi, bool norm, bool tall, int sa, int xf, bool rope) {
    switch (cpt) {
    case 1: return pick_tpr<M, 1>(tpr, fmt, swi, norm, tall, sa, xf, rope);
    case 2: return pick_tpr<M, 2>(tpr, fmt, swi, norm, tall, sa, xf, rope);
    case 3: return pick_tpr<M, 3>(tpr, fmt, swi, norm, tall, sa, xf, rope);
    default: return pick_tpr<M, 4>(tpr, fmt, swi, norm, tall, sa, xf, rope);
    }
}

}  // namespace

// The kernel instance for a supported call and the weight rows each of its
// blocks covers (block j: rows j * rows ..).
static Decode plan(const rq_qweight &w, bool swi, bool norm, int m, int sa, bool xf, bool rope, int *rows) {
    const int64_t N = w.n_out, K = w.k_in;
    const int C = (int)(K / 16);
    const int tpr = C <= 64 ? 64 : (C <= 128 ? 128 : 256);
    const int cpt = (int)cdiv(C, tpr);
    const int mt = m == 1 ? 1 : (m == 2 ? 2 : 4);
    const int fmt = w.format == RQ_Q_AFFINE_U8 ? 1 : 0;
    const bool tall = mt == 1 && !swi && fmt == 0 && N >= 16384;
    const int xr = !xf ? 0
                   : mt == 2 ? (N / 8 >= 512 ? 8 : 4)
                             : (N / 8 >= 1024 || (K > 4096 && N / 8 >= 512)) ? 8 : (N / 4 >= 1024 ? 4 : 2);
    const Decode d = mt == 1 ? pick_cpt<1>(cpt, tpr, fmt, swi, norm, tall && !rope, sa, xr, rope)
                             : mt == 2 ? pick_cpt<2>(cpt, tpr, fmt, swi, false, false, 0, xr, false)
                                       : pick_cpt<4>(cpt, tpr, fmt, swi, false, false, 0, false, false);
    *rows = d.r * (DT / tpr);
    return d;
}

// x: fp16 activations, or (nw != null, m = 1) the f32 row to RMS-normalise
// with the fp16 weight nw and epsilon eps, or (sa > 0, m = 1) the attention
// partials to combine (sa per head of attn_hd elements).
static int launch_decode(const rq_qweight &w, const rq_qweight *w2, const void *x, const _Float16 *nw, float eps,
                         void *y, int ymode, int m, hipStream_t s, int sa = 0, int attn_hd = 0, bool xf = false,
                         const RopeDecode *rd = nullptr) {
    const int64_t N = w.n_out, K = w.k_in;
    // f32 activations: m <= 2 and the plain row only; 32-bit offsets into X
    if (xf && (m > 2 || nw || sa || (int64_t)m * K * 4 > 0x7fffffffll)) return RQ_ERR_UNSUPPORTED;
    if (m < 1 || m > 4 || K % 16 != 0 || K > 16 * 256 * 4 || N > 0x7fffffff || !aligned(w.codes, 16) ||
        !aligned(x, 16) || (w.format == RQ_Q_AFFINE_U8 && (w.group % 16 != 0 || K % w.group != 0)))
        return RQ_ERR_UNSUPPORTED;
    if (w2 && (w2->format != w.format || w2->group != w.group || !aligned(w2->codes, 16)))
        return RQ_ERR_UNSUPPORTED;
    if (nw && (m != 1 || !aligned(nw, 16))) return RQ_ERR_UNSUPPORTED;
    if (sa && (m != 1 || w2 || nw || (sa != 1 && sa != 2 && sa != 4 && sa != 8) || attn_hd < 8 ||
               attn_hd % 8 != 0 || K % attn_hd != 0))
        return RQ_ERR_UNSUPPORTED;
    // the rotary epilogue: the normed m = 1 projection of whole heads, the
    // whole weight addressable with 32-bit offsets
    // (hd >= 32: a block's pairs, at most 12, cross at most one head boundary)
    if (rd && (!nw || m != 1 || w2 || sa || xf || rd->hd < 32 || rd->hd % 2 != 0 ||
               N != (int64_t)(rd->n_heads + 2 * rd->n_kv) * rd->hd || N * K > 0xffffffffll || !rd->pos ||
               !rd->rope || !rd->q || !rd->kc || !rd->vc))
        return RQ_ERR_UNSUPPORTED;
    int rows;
    const Decode d = plan(w, w2 != nullptr, nw != nullptr, m, sa, xf, rd != nullptr, &rows);
    const bool fx = nw || sa || xf;  // x is an f32 source
    const int64_t blocks = cdiv(N, rows);
    hipLaunchKernelGGL(d.fn, dim3((unsigned)blocks), dim3(DT), 0, s, (const uint8_t *)w.codes, w.scales, w.biases,
                       w2 ? (const uint8_t *)w2->codes : nullptr, w2 ? w2->scales : nullptr, w2 ? w2->biases : nullptr,
                       fx ? nullptr : (const _Float16 *)x, fx ? (const float *)x : nullptr, nw, eps, y, ymode, m,
                       (int)N, (int)K, w.group, attn_hd, rd ? *rd : RopeDecode{});
    RQ_LAUNCH_CHECK();
    return RQ_OK;
}

int launch_gemv_decode(const rq_qweight &w, const void *x, rq_dtype xt, void *y, rq_dtype yt, int m, hipStream_t s) {
    return launch_decode(w, nullptr, x, nullptr, 0.0f, y, yt == RQ_F16 ? kYF16 : kYF32, m, s, 0, 0, xt == RQ_F32);
}

int launch_gemv_decode_add(const rq_qweight &w, const void *x, float *y, int m, hipStream_t s) {
    return launch_decode(w, nullptr, x, nullptr, 0.0f, y, kYAdd, m, s);
}

int launch_gemv_decode_norm(const rq_qweight &w, const float *x, const _Float16 *nw, float eps, float *y,
                            hipStream_t s) {
    return launch_decode(w, nullptr, x, nw, eps, y, kYF32, 1, s);
}

int launch_swiglu_decode(const rq_qweight &gate, const rq_qweight &up, const void *x, rq_dtype xt, void *h, int m,
                         hipStream_t s) {
    return launch_decode(gate, &up, x, nullptr, 0.0f, h, kYF16, m, s, 0, 0, xt == RQ_F32);
}

int launch_swiglu_decode_norm(const rq_qweight &gate, const rq_qweight &up, const float *x, const _Float16 *nw,
                              float eps, void *h, hipStream_t s) {
    return launch_decode(gate, &up, x, nw, eps, h, kYF16, 1, s);
}

int launch_gemv_decode_qkv_rope(const rq_qweight &w, const float *x, const _Float16 *nw, float eps,
                                const RopeDecode &rd, hipStream_t s) {
    return launch_decode(w, nullptr, x, nw, eps, nullptr, kYF32, 1, s, 0, 0, false, &rd);
}

int launch_gemv_decode_attn_add(const rq_qweight &w, const float *partials, int n_split, int head_dim, float *y,
                                hipStream_t s) {
    return launch_decode(w, nullptr, partials, nullptr, 0.0f, y, kYAdd, 1, s, n_split, head_dim);
}

}  // namespace rq
