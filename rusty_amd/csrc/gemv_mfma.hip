// Decode dequant-GEMV on the matrix cores, 3 <= m <= 16 tokens:
// Y[m, n] = s[n] * sum_k X[m, k] * q[n, k].
//
// Still HBM-bound (every weight byte read once) but with 3-16 activation rows
// the per-byte arithmetic no longer fits the VALU budget of the dot2 kernel
// (m = 4, 4096x4096: 7.2 us there, 6.3 us here; m = 2 stays faster there),
// so the products go to v_mfma_f32_16x16x32_f16 (16 features x 16 tokens x 32
// k per instruction; MFMA throughput is far from the limit here):
//  * One block of NWV waves per 16 weight rows (SwiGLU: 8 gate + the same 8
//    up rows), or per two such row tiles where the launcher's measurements
//    favour it (tall weights, SwiGLU pairs): the activation block, re-read by
//    every block, is then read once for 32 rows.  Wave w takes the 256-k
//    batches w, w + NWV, ..., counted from a per-block rotation that
//    staggers the blocks' activation reads.
//  * Weights are loaded as 4 rows x 256 contiguous bytes per instruction
//    (lane chunk lane % 16 of row 4 i + lane / 16): against loading the MFMA
//    operand layout directly (16 rows x 64 B per instruction) the weight
//    streams 15-23 % faster.  Each wave then transposes its batch through its
//    own 4 KiB of LDS (ds_write_b128, then ds_read_b64 in operand layout, the
//    16-byte chunks XOR-swizzled by row) -- no barrier, the slice is private.
//  * Activations go straight from global memory into the B operand: lane
//    (fr = lane % 16, q = lane / 16) of MFMA j loads 16 bytes of token fr at
//    k = 256 b + 32 j + 8 q, the k its weight operand holds.
//  * All loads of a batch are issued before the first is used (a scheduling
//    barrier keeps the compiler from interleaving them with the conversions),
//    and the next batch's loads are in flight while the current batch is
//    multiplied.  Tokens >= m, rows >= N and k >= K read as zero.
//  * NWV = 8 where the one-tile grid is at most two blocks per CU and
//    K <= 4096 (one block per CU needs the eight waves' loads in flight), else
//    NWV = 4: more resident blocks per CU did better at K = 11008 or
//    N = 11008.
//  * The weight is expanded exactly in registers: XOR 0x80, v_perm_b32 under
//    exponent 0x64 (fp16 1152+q), v_pk_add_f16 -1152.
//  * The waves' 16x16 partial sums meet in LDS once; scale, fp16/f32 store
//    (SwiGLU: h = silu(g) * u).
#include "common.hpp"

#include <type_traits>

namespace rq {
namespace {

constexpr uint32_t kOOB = 0x80000000u;

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), 0, bytes, 0x00020000);
}
// aux bit 1 = non-temporal (the weights are streamed once), 0 = default caching
template <int AUX>
__device__ __forceinline__ uint4 bload(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const u32x4 v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, AUX));
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ uint32_t i8x2_to_f16x2(uint32_t u, uint32_t sel) {
    const uint32_t m = __builtin_amdgcn_perm(0x64646464u, u, sel);
    const h2_t v = __builtin_bit_cast(h2_t, m) - (h2_t){(_Float16)1152.0f, (_Float16)1152.0f};
    return __builtin_bit_cast(uint32_t, v);
}
// 8 signed int8 codes (two dwords) -> 8 exact fp16 values.
__device__ __forceinline__ half8 i8x8_to_half8(uint32_t lo, uint32_t hi) {
    const uint32_t a = lo ^ 0x80808080u, b = hi ^ 0x80808080u;
    uint4 r;
    r.x = i8x2_to_f16x2(a, 0x04010400u);
    r.y = i8x2_to_f16x2(a, 0x04030402u);
    r.z = i8x2_to_f16x2(b, 0x04010400u);
    r.w = i8x2_to_f16x2(b, 0x04030402u);
    return __builtin_bit_cast(half8, r);
}

__device__ __forceinline__ float silu(float v) { return v / (1.0f + expf(-v)); }

// 8 unsigned affine codes -> fp16 u*s + b, given c = b - 1024 s: v_perm_b32
// under exponent 0x64 gives fp16 1024 + u exactly, and fma(1024 + u, s, c) in
// f32 is rounded once to fp16 (v_fma_mix{lo,hi}_f16).
__device__ __forceinline__ uint32_t u8x2_affine(uint32_t u, uint32_t sel, float s, float c) {
    const h2_t m = __builtin_bit_cast(h2_t, __builtin_amdgcn_perm(0x64646464u, u, sel));
    const h2_t r = {(_Float16)__builtin_fmaf((float)m.x, s, c), (_Float16)__builtin_fmaf((float)m.y, s, c)};
    return __builtin_bit_cast(uint32_t, r);
}
__device__ __forceinline__ half8 u8x8_affine(uint32_t lo, uint32_t hi, float s, float c) {
    uint4 r;
    r.x = u8x2_affine(lo, 0x04010400u, s, c);
    r.y = u8x2_affine(lo, 0x04030402u, s, c);
    r.z = u8x2_affine(hi, 0x04010400u, s, c);
    r.w = u8x2_affine(hi, 0x04030402u, s, c);
    return __builtin_bit_cast(half8, r);
}

// One batch of a wave's operands: 256 k of the block's 16 weight rows, as
// loaded (4 rows x 256 B per instruction), and the activations of the 8 MFMAs
// that consume them (16 B per lane per MFMA, already in operand layout).
template <int FMT, bool XF, int RT = 1>
struct Batch {
    uint4 w[RT][4], x[XF ? 16 : 8];  // XF: 8 f32 activations (two loads) per MFMA
    // affine: the four group scales / biases of MFMA row fr (fp16 expansion);
    // affine with XF: those of output rows 4 q + r, r < 4 (applied after the MFMAs)
    float4 s[FMT == 1 && XF ? 4 : 1], b[FMT == 1 && XF ? 4 : 1];
};

// 8 unsigned affine codes -> their exact fp16 values u (0..255).
__device__ __forceinline__ half8 u8x8_exact(uint32_t lo, uint32_t hi) {
    const h2_t k = {(_Float16)1024.0f, (_Float16)1024.0f};
    uint4 r;
    r.x = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2_t, __builtin_amdgcn_perm(0x64646464u, lo, 0x04010400u)) - k);
    r.y = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2_t, __builtin_amdgcn_perm(0x64646464u, lo, 0x04030402u)) - k);
    r.z = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2_t, __builtin_amdgcn_perm(0x64646464u, hi, 0x04010400u)) - k);
    r.w = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2_t, __builtin_amdgcn_perm(0x64646464u, hi, 0x04030402u)) - k);
    return __builtin_bit_cast(half8, r);
}

// 8 f32 values x, scaled by 2^-sh (SC; exact) -> hi = fp16(x), lo =
// fp16(x - hi) (round to nearest even): hi + lo equals x to about 2^-22
// relative while |x| stays inside fp16's range.
template <bool SC = false>
__device__ __forceinline__ void f32x8_split(const uint4 a, const uint4 b, half8 &hi, half8 &lo, int sh = 0) {
    float f[8] = {__builtin_bit_cast(float, a.x), __builtin_bit_cast(float, a.y), __builtin_bit_cast(float, a.z),
                  __builtin_bit_cast(float, a.w), __builtin_bit_cast(float, b.x), __builtin_bit_cast(float, b.y),
                  __builtin_bit_cast(float, b.z), __builtin_bit_cast(float, b.w)};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        if constexpr (SC) f[e] = __builtin_amdgcn_ldexpf(f[e], -sh);
        hi[e] = (_Float16)f[e];
        lo[e] = (_Float16)(f[e] - (float)hi[e]);
    }
}

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
// Maximum over the 64 lanes, uniform across the wave.
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));   // quad_perm [1,0,3,2]
    v = fmaxf(v, dpp_f<0x4E>(v));   // quad_perm [2,3,0,1]
    v = fmaxf(v, dpp_f<0x141>(v));  // row_half_mirror
    v = fmaxf(v, dpp_f<0x140>(v));  // row_mirror: each 16-lane row holds its maximum
    const auto rl = [](float x, int l) {
        return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), l));
    };
    return fmaxf(fmaxf(rl(v, 0), rl(v, 16)), fmaxf(rl(v, 32), rl(v, 48)));
}

// SWI: SwiGLU gate/up pass -- the block's 16 weight rows are 8 gate rows (W)
// and the same 8 rows of the up weight (W2); it writes h = silu(g) * u (fp16).
// FMT 1: the reference's affine u8 codes with an f32 scale and bias per group
// of 64 along k (K % 256 == 0): each lane loads the four group scales and
// biases of its MFMA row for a batch (16 contiguous bytes each, beside the
// weight loads) and expands the codes to fp16 u*s + b before the MFMA; the
// epilogue then applies no row scale.
// XF: f32 activations (the reference's dtype), 32 bytes per lane per MFMA,
// each split into two fp16 terms multiplied separately; per-row codes enter
// as exact fp16 values, affine codes as exact u with the group's scale and
// bias applied in f32 after the MFMAs (u . x and the group sum of x).  A
// value past fp16's range makes its terms infinite and the batch's sums
// non-finite; such a batch (any lane of the wave) is multiplied again with
// every activation scaled by one wave-uniform power of two 2^-S that puts the
// batch's largest magnitude in [2^14, 2^15), its sums scaled back by 2^S.
// XFIRST: each batch's activation loads are issued before its weight loads
// (see launch_mfma).
// RT: row tiles per block (per-row codes, fp16 activations): tile t covers
// the block's rows t * RB .. (SwiGLU: 8 gate and the same 8 up rows each);
// every activation fragment a wave loads feeds the MFMAs of all RT tiles, so
// a block reads the activation block once for RT times the weight rows.
template <bool SWI, int NWV, int FMT = 0, bool XF = false, bool XFIRST = false, int RT = 1>
__global__ __launch_bounds__(NWV * 64) void k_gemv_mfma(const int8_t *__restrict__ W, const float *__restrict__ scales,
                                                  const int8_t *__restrict__ W2, const float *__restrict__ scales2,
                                                  const void *__restrict__ X, void *__restrict__ Yv, int y_f16,
                                                  int m_act, int N, int K, const float *__restrict__ biases,
                                                  const float *__restrict__ biases2) {
    static_assert(RT == 1 || (FMT == 0 && !XF), "row tiles: per-row codes, fp16 activations");
    static_assert(RT <= NWV, "one wave finishes each row tile");
    constexpr int RB = SWI ? 8 : 16;  // output rows per row tile
    __shared__ floatx4 red[NWV][RT][64];
    // per wave and tile: the 16 rows x 256 k of the batch being multiplied,
    // rows of 256 B with 16-byte chunk c of row r stored at chunk c ^ r
    __shared__ __attribute__((aligned(16))) uint8_t wt[NWV][RT][16 * 256];

    const int t = threadIdx.x, lane = t % 64;
    const int wave = __builtin_amdgcn_readfirstlane(t / 64);  // scalar: the batch loop branches uniformly
    const int fr = lane % 16, q = lane / 16;  // MFMA operand row (weight row / token) and lane group
    const int n0 = blockIdx.x * RB * RT;
    int rht[RT];  // rows of each tile (0 past the weight)
#pragma unroll
    for (int tt = 0; tt < RT; ++tt) rht[tt] = max(0, min(RB, N - (n0 + tt * RB)));
    const int rows_here = rht[0];
    // The row scales of this lane's outputs (rows 4 q + r), requested with the
    // first weight batch (below): loaded in the epilogue, each output waited
    // for its scale after the reduction (a round trip per output row on the
    // block's tail).
    float sc[RT][4], sc2[RT][4];
    auto load_scales = [&]() {
        if constexpr (FMT == 0) {
#pragma unroll
            for (int tt = 0; tt < RT; ++tt)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int f = 4 * q + r, row = (f < rht[tt] ? n0 + tt * RB + f : 0);
                    sc[tt][r] = scales[row];
                    if constexpr (SWI) sc2[tt][r] = scales2[row];
                }
        }
    };
    __amdgpu_buffer_rsrc_t rw[RT], rw2[RT];
#pragma unroll
    for (int tt = 0; tt < RT; ++tt) {
        const size_t r0 = (size_t)(n0 + tt * RB) * K;
        rw[tt] = make_rsrc(W + (rht[tt] ? r0 : 0), (uint32_t)rht[tt] * (uint32_t)K);
        rw2[tt] = make_rsrc((SWI ? W2 : W) + (rht[tt] ? r0 : 0), (uint32_t)rht[tt] * (uint32_t)K);
    }
    const auto rx = make_rsrc(X, (uint32_t)m_act * (uint32_t)K * (XF ? 4u : 2u));
    // Weight loads: instruction i covers rows 4 i + q, 256 contiguous bytes
    // each (lane chunk fr); SwiGLU: instructions 0-1 the gate rows 0-7, 2-3
    // the up rows 0-7.  A row past the weight, or k past K (which would fall
    // into the next row), reads as zero.
    const uint32_t xbase = ((uint32_t)fr * (uint32_t)K + 8u * (uint32_t)q) * (XF ? 4u : 2u);
    uint8_t *wl = wt[wave][0];
    const int nb = (K + 255) / 256;  // 256-k batches; wave w takes batches w, w + NWV, ...
    // ... counted from this block's rotation brot (mod nb).  Every block reads
    // all of X: unrotated, the blocks that share an XCD's L2 (consecutive
    // blocks go to the 8 XCDs in turn) all requested the same activation lines
    // at the same moment.  Block b is the (b / 8)-th of XCD b % 8; stepping the
    // rotation by 5 per block of an XCD and by 1 per XCD spreads them (MI355X,
    // us, unrotated -> rotated: m = 4 4096^2 6.41 -> 5.70, m = 16 8.03 -> 7.34,
    // m = 8 11008x4096 13.63 -> 12.70, m = 8 4096x11008 12.45 -> 11.30; with
    // X's loads taken out, 5.65 at every m).
    const int brot = (int)((blockIdx.x >> 3) * 5u + (blockIdx.x & 7u)) % nb;

    const int Gpr = K / 64;  // affine groups per row
    auto load = [&](Batch<FMT, XF, RT> &b, int bi) {
        int bb = bi + brot;
        bb -= bb >= nb ? nb : 0;
        const uint32_t k0 = (uint32_t)bb * 256u;
        const bool klive = k0 + 16u * (uint32_t)fr < (uint32_t)K;  // K % 16 == 0
        if constexpr (FMT == 1 && XF) {
            // output rows 4 q + r (SwiGLU: rows 0-7 gate, 8-15 up), four groups each
            const uint32_t bytes = (uint32_t)N * (uint32_t)Gpr * 4u;
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
                const int R = 4 * q + rr;
                const int r = SWI ? R % 8 : R;
                const bool up = SWI && R >= 8;
                const uint32_t off = r < rows_here && k0 < (uint32_t)K
                                         ? ((uint32_t)(n0 + r) * (uint32_t)Gpr + k0 / 64u) * 4u : kOOB;
                b.s[rr] = __builtin_bit_cast(float4, bload<0>(make_rsrc(up ? scales2 : scales, bytes), off));
                const float *bp = up ? biases2 : biases;
                b.b[rr] = bp ? __builtin_bit_cast(float4, bload<0>(make_rsrc(bp, bytes), off))
                             : float4{0.0f, 0.0f, 0.0f, 0.0f};
            }
        } else if constexpr (FMT == 1) {
            // MFMA row fr: weight row fr (SwiGLU: gate rows 0-7, up rows 8-15 of the same output rows)
            const int r = SWI ? fr % 8 : fr;
            const bool up = SWI && fr >= 8;
            const uint32_t bytes = (uint32_t)N * (uint32_t)Gpr * 4u;
            const uint32_t off = r < rows_here && k0 < (uint32_t)K
                                     ? ((uint32_t)(n0 + r) * (uint32_t)Gpr + k0 / 64u) * 4u : kOOB;
            b.s[0] = __builtin_bit_cast(float4, bload<0>(make_rsrc(up ? scales2 : scales, bytes), off));
            const float *bp = up ? biases2 : biases;
            b.b[0] = bp ? __builtin_bit_cast(float4, bload<0>(make_rsrc(bp, bytes), off)) : float4{0.0f, 0.0f, 0.0f, 0.0f};
        }
        auto wloads = [&]() {
#pragma unroll
            for (int tt = 0; tt < RT; ++tt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int r = SWI ? (4 * i + q) % 8 : 4 * i + q;  // row within the tile
                    const bool live = klive && r < rht[tt];
                    const uint32_t off = (uint32_t)r * (uint32_t)K + k0 + 16u * (uint32_t)fr;
                    b.w[tt][i] = bload<2>(SWI && i >= 2 ? rw2[tt] : rw[tt], live ? off : kOOB);
                }
        };
        auto xloads = [&]() {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const uint32_t k = k0 + 32u * (uint32_t)j;  // lane k = k + 8 q .. + 8
                const bool live = k + 8u * (uint32_t)q < (uint32_t)K;
                if constexpr (XF) {
                    b.x[2 * j] = bload<0>(rx, live ? xbase + k * 4u : kOOB);
                    b.x[2 * j + 1] = bload<0>(rx, live ? xbase + k * 4u + 16u : kOOB);
                } else {
                    b.x[j] = bload<0>(rx, live ? xbase + k * 2u : kOOB);
                }
            }
        };
        if constexpr (XFIRST) {
            xloads();
            wloads();
        } else {
            wloads();
            xloads();
        }
    };
    floatx4 acct[RT];
#pragma unroll
    for (int tt = 0; tt < RT; ++tt) acct[tt] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    floatx4 &acc = acct[0];
    // Transpose through the wave's LDS slice: lane (fr, q) of MFMA j takes the
    // 8 codes of row fr at k = 32 j + 8 q, the k order of its activations.
    // Only this wave touches the slice, and LDS operations of a wave complete
    // in order, so no barrier is needed around it.
    auto mma = [&](const Batch<FMT, XF, RT> &b) {
        uint2 at[RT][8];
#pragma unroll
        for (int tt = 0; tt < RT; ++tt) {
            uint8_t *wlt = wl + tt * (16 * 256);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = 4 * i + q;
                *reinterpret_cast<uint4 *>(wlt + r * 256 + ((fr ^ r) << 4)) = b.w[tt][i];
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int c = 2 * j + (q >> 1);
                at[tt][j] = *reinterpret_cast<const uint2 *>(wlt + fr * 256 + ((c ^ fr) << 4) + 8 * (q & 1));
            }
        }
        const uint2 *a = at[0];
        if constexpr (XF) {
            // f32 activations: the batch as loaded, then (rarely) again scaled
            auto mma_x = [&](auto scaled, int sh) {
                constexpr bool SC = decltype(scaled)::value;
                if constexpr (FMT == 1) {
                    // exact: per group g (MFMAs 2 g, 2 g + 1), t = u . x and xs =
                    // sum x over the group (ones as the weight operand), then
                    // acc += s . t + b . xs in f32 for output rows 4 q + r
                    half8 ones;
#pragma unroll
                    for (int e = 0; e < 8; ++e) ones[e] = (_Float16)1.0f;
#pragma unroll
                    for (int gi = 0; gi < 4; ++gi) {
                        floatx4 tg = {0.0f, 0.0f, 0.0f, 0.0f}, xg = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                        for (int jj = 0; jj < 2; ++jj) {
                            const int j = 2 * gi + jj;
                            const half8 ue = u8x8_exact(a[j].x, a[j].y);
                            half8 hi, lo;
                            f32x8_split<SC>(b.x[2 * j], b.x[2 * j + 1], hi, lo, sh);
                            tg = __builtin_amdgcn_mfma_f32_16x16x32_f16(ue, hi, tg, 0, 0, 0);
                            tg = __builtin_amdgcn_mfma_f32_16x16x32_f16(ue, lo, tg, 0, 0, 0);
                            xg = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, hi, xg, 0, 0, 0);
                            xg = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, lo, xg, 0, 0, 0);
                        }
#pragma unroll
                        for (int rr = 0; rr < 4; ++rr) {
                            const float sv = gi == 0 ? b.s[rr].x : gi == 1 ? b.s[rr].y : gi == 2 ? b.s[rr].z : b.s[rr].w;
                            const float bv = gi == 0 ? b.b[rr].x : gi == 1 ? b.b[rr].y : gi == 2 ? b.b[rr].z : b.b[rr].w;
                            const float t = SC ? __builtin_amdgcn_ldexpf(tg[rr], sh) : tg[rr];
                            const float xs = SC ? __builtin_amdgcn_ldexpf(xg[rr], sh) : xg[rr];
                            acc[rr] = __builtin_fmaf(sv, t, acc[rr]);
                            acc[rr] = __builtin_fmaf(bv, xs, acc[rr]);
                        }
                    }
                } else {
                    // x = hi + lo: the weight operand holds exact code values, so
                    // the two products together keep f32 accuracy
                    floatx4 t = acc;
                    if constexpr (SC) t = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const half8 av = i8x8_to_half8(a[j].x, a[j].y);
                        half8 hi, lo;
                        f32x8_split<SC>(b.x[2 * j], b.x[2 * j + 1], hi, lo, sh);
                        t = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, hi, t, 0, 0, 0);
                        t = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, lo, t, 0, 0, 0);
                    }
                    if constexpr (SC) {
#pragma unroll
                        for (int r = 0; r < 4; ++r) acc[r] += __builtin_amdgcn_ldexpf(t[r], sh);
                    } else {
                        acc = t;
                    }
                }
            };
            const floatx4 acc0 = acc;
            mma_x(std::false_type{}, 0);
            const bool bad = !(__builtin_isfinite(acc[0]) && __builtin_isfinite(acc[1]) &&
                               __builtin_isfinite(acc[2]) && __builtin_isfinite(acc[3]));
            if (__builtin_amdgcn_ballot_w64(bad) != 0) {  // wave-uniform
                float amax = 0.0f;
#pragma unroll
                for (int i = 0; i < 16; ++i)
                    amax = fmaxf(fmaxf(amax, fmaxf(fabsf(__builtin_bit_cast(float, b.x[i].x)),
                                                   fabsf(__builtin_bit_cast(float, b.x[i].y)))),
                                 fmaxf(fabsf(__builtin_bit_cast(float, b.x[i].z)),
                                       fabsf(__builtin_bit_cast(float, b.x[i].w))));
                // amax = f * 2^E, f in [0.5, 1); an infinite maximum gives E = 0,
                // and the infinity stays one
                const int sh = __builtin_amdgcn_frexp_expf(wave_max(amax)) - 15;
                acc = acc0;
                mma_x(std::true_type{}, sh);
            }
            return;
        }
        float sg[4], cg[4];  // affine: MFMA j covers k 32 j .. 32 j + 31, group j / 2 of the batch
        if constexpr (FMT == 1) {
            sg[0] = b.s[0].x; sg[1] = b.s[0].y; sg[2] = b.s[0].z; sg[3] = b.s[0].w;
            cg[0] = __builtin_fmaf(-1024.0f, sg[0], b.b[0].x);
            cg[1] = __builtin_fmaf(-1024.0f, sg[1], b.b[0].y);
            cg[2] = __builtin_fmaf(-1024.0f, sg[2], b.b[0].z);
            cg[3] = __builtin_fmaf(-1024.0f, sg[3], b.b[0].w);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
#pragma unroll
            for (int tt = 0; tt < RT; ++tt) {
                half8 av;
                if constexpr (FMT == 1) av = u8x8_affine(a[j].x, a[j].y, sg[j / 2], cg[j / 2]);
                else av = i8x8_to_half8(at[tt][j].x, at[tt][j].y);
                acct[tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, __builtin_bit_cast(half8, b.x[j]), acct[tt], 0,
                                                                   0, 0);
            }
        }
    };

    // Two batches alternate: the next one's loads are in flight while the
    // current one is multiplied.  Software-pipelined with a peeled tail so
    // that every load sits in the same straight-line block as the MFMAs that
    // consume it (a load whose only use lies behind a branch gets sunk past
    // the branch, and the prefetch is lost).  mb, the wave's batch count, is
    // wave-uniform.
    const int mb = (nb - wave + NWV - 1) / NWV;
    Batch<FMT, XF, RT> A, B;
    if (mb > 0) {
        load(A, wave);
        load_scales();
        int b = 0;
        for (; b + 2 < mb; b += 2) {
            load(B, wave + (b + 1) * NWV);
            __builtin_amdgcn_sched_barrier(0);  // issue every load before the conversions
            mma(A);
            load(A, wave + (b + 2) * NWV);
            __builtin_amdgcn_sched_barrier(0);
            mma(B);
        }
        if (b + 1 < mb) {
            load(B, wave + (b + 1) * NWV);
            __builtin_amdgcn_sched_barrier(0);
            mma(A);
            mma(B);
        } else {
            mma(A);
        }
    } else {
        // no batch for this wave (nb <= wave: K <= 256 wave), which may still
        // finish a row tile below (wave t finishes tile t): its scales all the same
        load_scales();
    }

    // acct[t] = D[feature 4 q + r][token fr] of tile t, partial over this
    // wave's groups; wave t finishes tile t.
#pragma unroll
    for (int tt = 0; tt < RT; ++tt) red[wave][tt][lane] = acct[tt];
    __syncthreads();
#pragma unroll
    for (int tt = 0; tt < RT; ++tt) {
        if (wave != tt) continue;
        const int nt = n0 + tt * RB, rh = rht[tt];
        floatx4 v = red[0][tt][lane];
#pragma unroll
        for (int w = 1; w < NWV; ++w) {
            const floatx4 o = red[w][tt][lane];
            v[0] += o[0];
            v[1] += o[1];
            v[2] += o[2];
            v[3] += o[3];
        }
        const int m = fr;
        if constexpr (SWI) {
            // gate rows 0..7 sit in lane groups 0-1, up rows 8..15 in groups 2-3
            red[0][tt][lane] = v;
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            const floatx4 u = red[0][tt][(lane + 32) % 64];
            if (q < 2 && m < m_act) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int f = 4 * q + r;
                    if (f < rh) {
                        const float h = FMT == 1 ? silu(v[r]) * u[r] : silu(v[r] * sc[tt][r]) * (u[r] * sc2[tt][r]);
                        reinterpret_cast<_Float16 *>(Yv)[(size_t)m * N + nt + f] = (_Float16)h;
                    }
                }
            }
        } else if (m < m_act) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int f = 4 * q + r;
                if (f < rh) {
                    const float y = FMT == 1 ? v[r] : v[r] * sc[tt][r];
                    const size_t o = (size_t)m * N + nt + f;
                    if (y_f16) reinterpret_cast<_Float16 *>(Yv)[o] = (_Float16)y;
                    else reinterpret_cast<float *>(Yv)[o] = y;
                }
            }
        }
    }
}

}  // namespace

static int launch_mfma(const rq_qweight &w, const rq_qweight *w2, const void *x, rq_dtype xt, void *y, rq_dtype yt,
                       int m, hipStream_t s) {
    const int64_t N = w.n_out, K = w.k_in;
    const bool affine = w.format == RQ_Q_AFFINE_U8, xf = xt == RQ_F32;
    // 32-bit buffer offsets: 16 activation rows of K values must stay below 2^31 bytes.
    if (m < 1 || m > 16 || K % 16 != 0 || K > (1 << 24) / (xf ? 2 : 1) || N > 0x7fffffff || !aligned(w.codes, 16) ||
        !aligned(x, 16))
        return RQ_ERR_UNSUPPORTED;
    if (affine && (w.group != 64 || K % 256 != 0 || (int64_t)N * (K / 64) * 4 > 0xffffffffll)) return RQ_ERR_UNSUPPORTED;
    if (w2 && (w2->format != w.format || !aligned(w2->codes, 16) || (affine && w2->group != w.group)))
        return RQ_ERR_UNSUPPORTED;
    // Two row tiles per block (per-row codes, fp16 activations): each block
    // reads the activation block (m x K fp16, re-read by every block) once for
    // twice the weight rows.  Taken where it measured faster (us, rotating
    // copies past the Infinity Cache; one tile -> two):
    //   gate/up pairs 11008 x 4096 (1376 tiles), 4 waves: SwiGLU m = 4 / 8 / 16
    //     30.1 -> 29.7, 33.1 -> 31.5, 44.6 -> 37.5 (whole MLP)
    //   8192 x 4096 (512 tiles), 8 waves: m = 8 10.27 -> 8.42
    //   11008 x 4096 (688 tiles), 4 waves: m = 16 16.86 -> 15.56, but
    //     m = 4 / 8 11.61 -> 13.18, 12.55 -> 13.9 (344 blocks leave the second
    //     round of the grid a third full); 11264 x 2048 likewise
    //   4096 x 4096 (256 tiles): 128 blocks, m = 8 6.04 -> 7.33
    const int64_t rows_tile = w2 ? 8 : 16, blocks1 = cdiv(N, rows_tile);
    const bool two = !affine && !xf &&
                     (w2 ? blocks1 >= 512 : (blocks1 > 256 && blocks1 <= 512) || (m > 8 && blocks1 > 512));
    const int64_t blocks = two ? cdiv(N, 2 * rows_tile) : blocks1;
    auto go = [&](auto nwv, auto fmt, auto xfc, auto rtc) {
        constexpr int NW = decltype(nwv)::value, F = decltype(fmt)::value, RT = decltype(rtc)::value;
        constexpr bool XF = decltype(xfc)::value;
        if (w2)
            hipLaunchKernelGGL((k_gemv_mfma<true, NW, F, XF, false, RT>), dim3((unsigned)blocks), dim3(NW * 64), 0, s,
                               (const int8_t *)w.codes, w.scales, (const int8_t *)w2->codes, w2->scales, x, y, 1, m,
                               (int)N, (int)K, w.biases, w2->biases);
        else {
            constexpr bool XFP = NW == 8 && F == 0 && !XF;  // the activation-first variant exists
            if (XFP && m >= 8)
                hipLaunchKernelGGL((k_gemv_mfma<false, NW, F, XF, XFP, RT>), dim3((unsigned)blocks), dim3(NW * 64), 0,
                                   s, (const int8_t *)w.codes, w.scales, nullptr, nullptr, x, y, yt == RQ_F16 ? 1 : 0, m,
                                   (int)N, (int)K, w.biases, nullptr);
            else
                hipLaunchKernelGGL((k_gemv_mfma<false, NW, F, XF, false, RT>), dim3((unsigned)blocks), dim3(NW * 64), 0,
                                   s, (const int8_t *)w.codes, w.scales, nullptr, nullptr, x, y, yt == RQ_F16 ? 1 : 0, m,
                                   (int)N, (int)K, w.biases, nullptr);
        }
    };
    auto go_fmt = [&](auto nwv, auto xfc) {
        // (affine codes with f32 activations run 4 waves, see `wide`: the
        // 8-wave variant is not built)
        constexpr bool aff_ok = decltype(nwv)::value == 4 || !decltype(xfc)::value;
        if (affine) {
            if constexpr (aff_ok) go(nwv, std::integral_constant<int, 1>{}, xfc, std::integral_constant<int, 1>{});
        }
        else if (two) go(nwv, std::integral_constant<int, 0>{}, std::false_type{}, std::integral_constant<int, 2>{});
        else go(nwv, std::integral_constant<int, 0>{}, xfc, std::integral_constant<int, 1>{});
    };
    auto go_x = [&](auto nwv) {
        if (xf) go_fmt(nwv, std::true_type{});
        else go_fmt(nwv, std::false_type{});
    };
    // Activations before weights in each batch (XFIRST) for per-row codes and
    // fp16 x at 8 waves and m >= 8, where the block's activation block (m x K
    // fp16, re-read by every block) is the longest-waiting load: 4096^2 m = 8 /
    // 12 / 16 6.03 -> 5.90, 6.68 -> 6.43, 7.34 -> 7.0 us.  Slower at m = 4
    // (5.70 -> 5.81), at 4 waves (11008 x 4096 m = 16 16.5 -> 17.1) and for
    // affine codes (m = 16 7.9 -> 8.4).
    // affine codes with f32 activations hold four scale and bias vectors per
    // batch: at 8 waves (256 VGPRs each) they spill, at 4 they fit
    const bool wide = K <= 4096 && blocks1 <= 512 && !(affine && xf);
    if (wide) go_x(std::integral_constant<int, 8>{});
    else go_x(std::integral_constant<int, 4>{});
    RQ_LAUNCH_CHECK();
    return RQ_OK;
}

int launch_gemv_mfma(const rq_qweight &w, const void *x, rq_dtype xt, void *y, rq_dtype yt, int m, hipStream_t s) {
    return launch_mfma(w, nullptr, x, xt, y, yt, m, s);
}

int launch_swiglu_mfma(const rq_qweight &gate, const rq_qweight &up, const void *x, rq_dtype xt, void *h, int m,
                       hipStream_t s) {
    return launch_mfma(gate, &up, x, xt, h, RQ_F16, m, s);
}

}  // namespace rq
