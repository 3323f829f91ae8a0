// Prefill dequant-GEMM for gfx950: Y[m, n] = s[n] * sum_k X[m, k] * q[n, k].
//
// Replaces, for a prompt of many tokens, the reference's f32 `matmul_tiled`
// (rusty-backend/src/kernels.wgsl:7-54) on a load-time-dequantized weight
// (kernels.wgsl:379-400).  MFMA-bound: 2*M*N*K flops over 1 B/weight + 2 B/act.
//
// Design (each choice measured on MI355X):
//  * Block tile BM tokens x BN features, 64 k per step, NW waves as KG
//    k-groups of (NW/KG/WGN) x WGN waves; each wave (BM/(NW/KG/WGN)) x
//    (BN/WGN) outputs as 32x32 tiles of v_mfma_f32_32x32x16_f16 (16x16x32
//    keeps the MFMA pipe only ~50% busy).  MFMA A = W (32 features x 16 k),
//    B = X^T (16 k x 32 tokens): a lane's accumulator holds runs of 4
//    consecutive features of one token (8-byte fp16 stores).  The 256x128
//    and 128x128 tiles run 8 waves (two per SIMD: while one wave of a SIMD
//    waits on its DMA issue or LDS reads the other issues MFMAs) as two
//    k-groups: group g multiplies k16 slices 2g, 2g+1 of every stage, so each
//    wave covers 128 (or 64) tokens x 64 features with the fragment reads and
//    int8 expansion of half a stage, and the groups add their partial sums
//    once through the ring at the end.  Against one group of 128x32 waves
//    the LDS fragment reads per MFMA fall from 1.1 to 0.63 KiB at the same
//    expansion work: 2048x4096x11008 178.8 -> 172.6 us, m = 768 and 1024 at
//    N = K = 4096 (128x128 tile, against 4 waves) 38.3 -> 35.5 us and
//    42.9 -> 40.6 us; 2048x4096x4096 unchanged.
//    The 128x64 and 64x64 tiles run 4 waves as two k-groups of 2 (2 x 1
//    along features), each wave all the tile's tokens x 32 features (KSPLIT_M:
//    the groups finish alternate token tiles): every expanded W fragment then
//    feeds 2 (64x64) or 4 (128x64) MFMAs instead of 1 or 2.  At these tiles
//    the int8 expansion, not the MFMAs, had set the pace (a timing-only copy
//    without it ran 512x2048x5632 24.2 -> 17.4 us): 512x2048x5632 24.2 ->
//    ~20.0, 512x2048x2048 10.7 -> 8.6, 256x4096x4096 18.7 -> 14.5,
//    64x4096x4096 (split K) 9.5 -> 8.5, 512x4096x11008 (128x64) 63 -> 57 us.
//  * Staging is direct-to-LDS DMA (buffer_load_dwordx4 ... lds): each wave
//    moves 1 KiB units from global memory straight into LDS, so tiles never
//    pass through VGPRs or ds_write (register staging measured ~10% slower,
//    limited by LDS write issue).  The weight stays int8 in LDS (half the
//    bytes) and is expanded to fp16 when a wave reads its fragment:
//    XOR 0x80 -> q+128, v_perm_b32 under exponent 0x64 -> fp16 1152+q,
//    v_pk_add_f16 -1152 -> q (exact).
//  * What staging costs is the cache lines each DMA touches, not its bytes:
//    one 1 KiB unit of X covers 8 rows x 128 B (8 whole lines); a unit of W
//    at 64 k per step covered 16 rows x 64 B (16 half lines), and W staging
//    measured 2x X's cost per unit.  So the large tiles (W2) stage W two
//    k-steps at a time: 128 B of each row, whole lines, into a ring of two
//    pairs beside the X ring (the same LDS as four single steps), every other
//    iteration.  A lane then reads its W fragment as one 16-byte piece that
//    covers both of its k16 slices (a k permutation matched by the X reads),
//    so every fragment read is a conflict-free ds_read_b128 (W reads were
//    ds_read_b64 with a 2-way bank conflict).  256x128: 66.0 -> 64.5 us.
//  * Measured with the same instruction stream and zero activations, the
//    kernel runs 27 % faster (61.7 -> 45.1 us at 2048x4096x4096; zero
//    weights 48.2): with random fp16 data the chip's power limit, not the
//    schedule, sets the clock.  Deeper rings (6 X stages, or 3 W pairs) and
//    64x128 wave tiles (less LDS, twice the int8 expansion) measured equal or
//    slower.
//  * An S-stage LDS ring, one barrier per k-step.  The loads of a stage are
//    waited for with an explicit vmcnt (loads retire in order), so the DMA of
//    the next steps stays in flight.  PINGPONG: the fragments of step k+1 are
//    read into registers while the MFMAs of step k run.
//  * LDS layouts are XOR-swizzled per 16-byte chunk (the DMA writes 1 KiB
//    contiguous per wave, so padding is impossible): X rows and W-pair rows
//    (128 B) put chunk c at c ^ ((row >> 1) & 7), single-step W rows (64 B) at
//    c ^ ((row >> 2) & 3), which spreads the 32 rows an MFMA operand reads
//    over the banks.
//  * Rows past M/N and k past K are offsets past the buffer resource and read
//    as zero: no branches around the loads; the k loop is padded to the ring
//    period with zero steps.
//  * XCD-aware tile order (tile_of): the blocks one XCD runs together cover a
//    group of GM token panels x the matching feature panels, so their X and
//    W panels are shared in that XCD's L2.
#include <algorithm>
#include <type_traits>

#include "common.hpp"
#include "lds_dma.hpp"

namespace rq {
namespace {

constexpr uint32_t kOOB = 0x80000000u;  // any offset past a buffer resource reads zero

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

// Split-K workspace layout: partial sums per (tile, split) slot of BM x BN f32;
// one arrival counter per tile on its own 128-byte line.
constexpr int kSkCounterStride = 32;
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

// 8 unsigned affine codes u (two dwords) -> fp16 u*s + b, given c = b - 1024 s:
// v_perm_b32 under exponent 0x64 gives fp16 1024 + u exactly, and
// v_fma_mix{lo,hi}_f16 evaluates fma(1024 + u, s, c) in f32 with one rounding
// to fp16 (this translation unit flushes f32 denormals, which lets the
// compiler select the mixed-precision FMA: 1.5 VALU per weight).
__device__ __forceinline__ uint32_t u8x2_affine(uint32_t u, uint32_t sel, float s, float c) {
    const h2_t m = __builtin_bit_cast(h2_t, __builtin_amdgcn_perm(0x64646464u, u, sel));
    const h2_t r = {(_Float16)__builtin_fmaf((float)m.x, s, c), (_Float16)__builtin_fmaf((float)m.y, s, c)};
    return __builtin_bit_cast(uint32_t, r);
}
__device__ __forceinline__ half8 u8x8_affine(uint2 w, float s, float c) {
    uint4 r;
    r.x = u8x2_affine(w.x, 0x04010400u, s, c);
    r.y = u8x2_affine(w.x, 0x04030402u, s, c);
    r.z = u8x2_affine(w.y, 0x04010400u, s, c);
    r.w = u8x2_affine(w.y, 0x04030402u, s, c);
    return __builtin_bit_cast(half8, r);
}

// Tile order: consecutive blocks go round-robin to the 8 XCDs, so block b
// runs on XCD b % 8; it takes position L = (b % 8) * (tiles / 8) + b / 8 of
// a group-M order (GM m-tiles per group, n-tiles across, m fastest within a
// group).  The 32 concurrent tiles of one XCD then cover GM token panels x
// 32/GM feature panels, so both X and W panels are reused in that XCD's L2.
__device__ __forceinline__ void tile_of(int b, int tiles_m, int tiles_n, int gm, int &tm, int &tn) {
    const int tiles = tiles_m * tiles_n;  // b < tiles
    const int L = (tiles % 8 == 0) ? (b % 8) * (tiles / 8) + b / 8 : b;
    const int per_group = gm * tiles_n;
    const int first_m = (L / per_group) * gm;
    const int gsize = min(gm, tiles_m - first_m);
    const int r = L % per_group;
    tm = first_m + r % gsize;
    tn = r / gsize;
}

// FMT 0: per-row int8 codes, scales[n] applied in the epilogue.  FMT 1: the
// reference's affine u8 codes with a scale and bias per group of G (a multiple
// of 64) along k; `scales` then holds them transposed, per group g a row of N
// scales s and a row of N offsets c = b - 1024 s (gemm_affine_prep), so a
// k-step's values for the block's BN features are contiguous: each wave
// stages 64 of them per k-step (one 4-byte DMA per lane) beside its X stage,
// and the weight is expanded to fp16 u*s + b while the fragments are read.
// PAIR, SwiGLU's gate and up (n_split = I rows each, N = 2 I; affine codes
// stage their scales from the gate's table and the up weight's, scalesb):
// tile column block tn covers rows [j0, j0 + BN/2) of both weights, j0 =
// tn * BN/2 -- the gate (W, scales) in tile columns [0, BN/2), the up weight
// (Wb, scalesb) in [BN/2, BN) -- and the epilogue writes h = silu(g) * u
// (g and u rounded to fp16 first, as a separate silu*mul pass over stored
// g and u would see them) to Yv, fp16 [M][I] (I % 8 == 0).  Only the two
// large tiles are built with it (the smaller ones run near the SGPR limit).
// ROPE (BN = 64 = head_dim, per-row codes, no split): the tile's 64 features
// are one head of the packed q/k/v output, and the epilogue applies the
// rotary embedding to q and k heads -- o[d] = a c - b s, o[d + 32] = a s + b c
// for a, b the f32 results at d and d + 32 -- and writes q (Yv) and the K and
// V caches (RopeOut) in fp16 instead of the f32 product.
template <int BM, int BN, bool PINGPONG, int S, int NW, int WGN, int KG = 1, bool W2 = false, int FMT = 0,
          bool PAIR = false, bool ROPE = false>
__global__ __launch_bounds__(64 * NW) void k_gemm_rowwise(const uint8_t *__restrict__ W, const float *__restrict__ scales,
                                                     const _Float16 *__restrict__ X, void *__restrict__ Yv,
                                                     int y_f16, int M, int N, int K, int tiles_m, int tiles_n,
                                                     int gm, int splits, float *__restrict__ skw,
                                                     int *__restrict__ skc, int group, const uint8_t *__restrict__ Wb,
                                                     const float *__restrict__ scalesb, int n_split, RopeOut ro,
                                                     const float *__restrict__ xscale) {
    static_assert(!ROPE || (BN == 64 && !PAIR), "rotary epilogue: one 64-wide head per tile");
    // KG k-groups of NW/KG waves: group g takes k16 slices [g*K16, (g+1)*K16)
    // of every 64-k stage, so a wave tile covers KG times the outputs for the
    // same fragment bytes; the groups' partial sums meet in LDS at the end.
    constexpr int WPG = NW / KG;   // waves per k-group
    constexpr int K16 = 4 / KG;    // 16-k slices per wave per stage
    constexpr int WGM = WPG / WGN; // wave grid: WGM along tokens, WGN along features
    constexpr int TM = BM / WGM, TN = BN / WGN, FM = TM / 32, FN = TN / 32;
    // The two k-groups finish disjoint halves of the wave tile: the feature
    // tiles i % 2 == kg, or (KSPLIT_M, a wave tile one feature tile wide) the
    // token tiles j % 2 == kg.
    constexpr bool KSPLIT_M = KG == 2 && FN % 2 != 0;
    static_assert(KG == 1 || (KG == 2 && (FN % 2 == 0 || FM % 2 == 0)), "two k-groups split the finishing work");
    // W2: the weight is staged two k-steps at a time (128-byte row pieces, whole
    // cache lines) in a ring of two pairs beside an S-stage X ring.
    static_assert(!W2 || (KG == 2 && PINGPONG && S == 4), "W pairs: two k-groups, ping-pong, 4 X stages");
    constexpr int XUW = BM * 128 / 1024 / NW;
    constexpr int WUW = W2 ? BN * 128 / 1024 / NW : BN * 64 / 1024 / NW;  // 1 KiB DMA units per wave
    static_assert(FM >= 1 && FN >= 1 && XUW >= 1 && WUW >= 1, "tile too small");
    static_assert(FMT == 0 || 2 * BN <= 64 * NW, "affine: one 4-byte DMA per lane covers a k-step's s and c");
    constexpr int XSTRIDE = W2 ? BM * 128 : BM * 128 + BN * 64;  // bytes between X stages
    constexpr int SCB = FMT == 1 ? 64 * NW * 4 : 0;  // affine s and c of one k-step (per X stage)
    constexpr int RING_X = W2 ? S * BM * 128 + 2 * BN * 128 : S * (BM * 128 + BN * 64);  // X and W stages
    constexpr int RING_K = RING_X + S * SCB;  // k-loop stages
    // the epilogue reuses the ring to stage a tile of f32 (or fp16) rows
    constexpr int RING = RING_K > BM * (BN * 4 + 16) ? RING_K : BM * (BN * 4 + 16);
    static_assert(S >= 3 && RING <= 160 * 1024, "ring does not fit in LDS");
    constexpr int XOPS = XUW + (FMT == 1 ? 1 : 0);  // DMA ops per wave issued with each X stage
    constexpr int NOUT = XOPS + WUW;  // DMA ops per wave per k-step (W2: W on odd steps only)

    __shared__ __attribute__((aligned(1024))) uint8_t ring[RING];

    // Split-K (splits > 1): block b multiplies tile b % tiles over the split
    // b / tiles of its k-steps; the tile's last block to finish adds every
    // split's partial sums (see below).
    const int tiles = tiles_m * tiles_n, tile = blockIdx.x % tiles, split = blockIdx.x / tiles;
    int tm, tn;
    tile_of(tile, tiles_m, tiles_n, gm, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    // the wave index as a uniform (scalar) value: LDS bases and DMA offsets
    // derived from it stay in SGPRs instead of being re-derived every k-step
    const int t = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(t / 64), lane = t % 64;
    const int kg = wave / WPG, wq = wave % WPG;
    const int wm = wq / WGN, wn = wq % WGN;
    const int fr = lane % 32, h = lane / 32;
    // whether this wave finishes output tile (i, j) of its wave tile
    auto mine = [&](int i, int j) { return KG == 1 || (KSPLIT_M ? j % 2 == kg : i % 2 == kg); };
    const int nk_all = K / 64, ks = (nk_all + splits - 1) / splits;
    const int k0 = split * ks, nk = min(ks, nk_all - k0);  // this block's k-steps [k0, k0 + nk)

    // PAIR: the tile's first row in each weight, the rows per weight (and h's row length)
    constexpr int HB = BN / 2;
    const int nw0 = PAIR ? n0 / 2 : n0;
    const int NL = PAIR ? n_split : N;
    // (PAIR: the compiler keeps some of these uniform values in VGPRs)
    const auto rx = PAIR ? make_rsrc_s(X + (size_t)m0 * K, (uint32_t)min(BM, M - m0) * (uint32_t)K * 2u)
                         : make_rsrc(X + (size_t)m0 * K, (uint32_t)min(BM, M - m0) * (uint32_t)K * 2u);
    const auto rw = PAIR ? make_rsrc_s(W + (size_t)nw0 * K, (uint32_t)min(HB, NL - nw0) * (uint32_t)K)
                         : make_rsrc(W + (size_t)n0 * K, (uint32_t)min(BN, N - n0) * (uint32_t)K);
    const auto rwb = PAIR ? make_rsrc_s(Wb + (size_t)nw0 * K, (uint32_t)min(HB, NL - nw0) * (uint32_t)K) : rw;
    // affine: lane l of wave w stages value i = 64 w + l of [s | c] for the
    // block's features (rows past N and lanes past 2 BN read zero); the
    // transposed scales hold 2 NL floats per group.  PAIR: the features of
    // the tile's second half are up rows, whose table is scalesb; 64 divides
    // HB, so each wave's 64 values come from one table (the DMA's buffer
    // descriptor is wave-uniform).
    const int gstep = FMT == 1 ? group / 64 : 1;  // k-steps per scale group
    const bool up_w = PAIR && ((wave * 64) % BN) >= HB;  // wave-uniform
    const auto rsc = make_rsrc(up_w ? static_cast<const float *>(scalesb) : scales,
                               FMT == 1 ? (uint32_t)(K / group) * (uint32_t)NL * 8u : 0u);
    uint32_t scoff = kOOB;
    if constexpr (FMT == 1) {
        const int i = wave * 64 + lane, f = i < BN ? i : i - BN;
        const int n = nw0 + (up_w ? f - HB : f);  // row of its weight (PAIR: of the gate or the up weight)
        if (i < 2 * BN && n < NL) scoff = (uint32_t)((i < BN ? 0 : NL) + n) * 4u;
    }

    // Source offsets (k = 0) of this lane in each of the wave's DMA units,
    // swizzled so LDS chunk s of row r holds global chunk s ^ f(r).
    uint32_t xoff[XUW], woff[WUW];
#pragma unroll
    for (int q = 0; q < XUW; ++q) {
        const int row = (wave * XUW + q) * 8 + lane / 8, s = lane % 8;
        xoff[q] = ((uint32_t)row * K + (uint32_t)(s ^ ((row >> 1) & 7)) * 8) * 2u;
    }
#pragma unroll
    for (int q = 0; q < WUW; ++q) {
        if constexpr (W2) {
            // 8 rows x 128 bytes (two k-steps) per unit, chunk s of row r holding
            // global chunk s ^ ((r >> 1) & 7)
            // (PAIR: tile rows from HB on are rows of the up weight)
            const int row = (wave * WUW + q) * 8 + lane / 8, s = lane % 8;
            const int wr = PAIR && row >= HB ? row - HB : row;
            woff[q] = (uint32_t)wr * K + (uint32_t)(s ^ ((row >> 1) & 7)) * 16;
        } else {
            const int row = (wave * WUW + q) * 16 + lane / 4, s = lane % 4;
            woff[q] = (uint32_t)row * K + (uint32_t)(s ^ ((row >> 2) & 3)) * 16;
        }
    }
    // LDS address of the ring, taken once: per-stage addresses are then plain
    // scalar sums (a generic-to-LDS pointer cast in the loop costs a null check
    // and a readfirstlane per DMA)
    const uint32_t ring_lds = (uint32_t)(uintptr_t)(lds_void *)&ring[0];
    auto dma = [&](int stage, int kt) {
        const bool live = kt < nk;
        kt += k0;
        const uint32_t sx = ring_lds + (uint32_t)stage * (uint32_t)XSTRIDE;
        if constexpr (FMT == 1)
            dma4(rsc, ring_lds + (uint32_t)(RING_X + stage * SCB + wave * 256),
                 live && scoff != kOOB ? scoff + (uint32_t)(kt / gstep) * (uint32_t)NL * 8u : kOOB);
#pragma unroll
        for (int q = 0; q < XUW; ++q) dma16(rx, sx + (uint32_t)(wave * XUW + q) * 1024u, live ? xoff[q] + kt * 128 : kOOB);
        if constexpr (!W2) {
            const uint32_t sw = sx + (uint32_t)(BM * 128);  // the W tile follows the X tile
#pragma unroll
            for (int q = 0; q < WUW; ++q) dma16(rw, sw + (uint32_t)(wave * WUW + q) * 1024u, live ? woff[q] + kt * 64 : kOOB);
        }
    };
    // W2: the weight of steps kt, kt + 1 (kt even) into pair slot `pair`.  The
    // second step past this block's k range reads the next bytes of the row
    // (or zeros past the weight): finite codes that only meet zero activations.
    auto dma_w = [&](int pair, int kt) {
        const bool live = kt < nk;
        kt += k0;
        const uint32_t sw = ring_lds + (uint32_t)(S * BM * 128) + (uint32_t)pair * (uint32_t)(BN * 128);
#pragma unroll
        for (int q = 0; q < WUW; ++q)
            dma16(PAIR && (wave * WUW + q) * 8 >= HB ? rwb : rw, sw + (uint32_t)(wave * WUW + q) * 1024u,
                  live ? woff[q] + kt * 64 : kOOB);
    };

    floatx16 acc[FN][FM];
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    // The per-feature scales of the outputs this wave finishes (feature tile i
    // = FKG io + (kg, or 0 with KSPLIT_M), features fl + r of each 8-row group
    // g), requested before the k loop: loaded by the epilogue, they cost a
    // round trip on every block's tail.  Past the weight's rows: a valid row,
    // zeroed at use.
    constexpr int FKG = KSPLIT_M ? 1 : KG;   // feature-tile stride of the finished tiles
    constexpr int FNO = FN / FKG;            // feature tiles this wave finishes
    constexpr int FMO = KSPLIT_M ? FM / 2 : FM;  // token tiles this wave finishes of each
    auto feat = [&](int io, int g) { return wn * TN + (FKG * io + (KSPLIT_M ? 0 : kg)) * 32 + 8 * g + h * 4; };
    auto wrow = [&](int fl) { return nw0 + (PAIR && fl >= HB ? fl - HB : fl); };
    float esc[FNO][4][4];
    if constexpr (FMT == 0) {
#pragma unroll
        for (int io = 0; io < FNO; ++io)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int fl = feat(io, g);
                const float *__restrict__ scl = PAIR && fl >= HB ? scalesb : scales;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int wr = wrow(fl) + r;
                    esc[io][g][r] = scl[wr < NL ? wr : 0];
                }
            }
    }
    // f32 activations cast with a per-row power of two (xscale: 2^e per token
    // row, the X rows holding x * 2^-e): the factor of every token row this
    // lane's outputs cover, multiplied in by the epilogue (exact; 1 without
    // xscale).  Requested here for the same reason as the scales.
    float tfac[FM];
#pragma unroll
    for (int j = 0; j < FM; ++j) {
        const int tr = m0 + wm * TM + j * 32 + fr;
        tfac[j] = xscale ? xscale[tr < M ? tr : M - 1] : 1.0f;
    }
    // ROPE: the (cos, sin) of the pairs 4 (t % 8) .. + 3 at the positions of
    // the tile rows this thread writes (32 ps + t / 8), requested here for the
    // same reason (also for a v head, which does not use them: no branch)
    constexpr int RRP = NW * 64 / 8;  // epilogue rows per pass: 8 threads per row
    float4 rcs[ROPE ? BM / RRP : 1][2];
    if constexpr (ROPE) {
#pragma unroll
        for (int ps = 0; ps < BM / RRP; ++ps) {
            const int sr = min(m0 + ps * RRP + t / 8, M - 1);
            const float4 *rp = reinterpret_cast<const float4 *>(ro.rope + (size_t)(ro.p0 + sr) * 32 + 4 * (t % 8));
            rcs[ps][0] = rp[0];
            rcs[ps][1] = rp[1];
        }
    }

    // A k-step's fragments: raw int8 W (expanded just before the MFMA) and fp16 X.
    // W2 reads a lane's W as one 16-byte piece covering both of its k16 slices
    // (a k permutation: slice kl takes bytes 8 kl .. 8 kl + 7 of the piece at
    // k = 32 kg + 16 h, and X supplies the same k), so every fragment read is a
    // conflict-free ds_read_b128.
    struct Frag {
        uint2 w[K16][FN];
        half8 x[K16][FM];
        float s[FMT == 1 ? FN : 1], c[FMT == 1 ? FN : 1];  // affine: the scale and offset of each W row
    };
    auto fetch = [&](int stage, int kt, Frag &f) {
        const uint8_t *sx = ring + stage * XSTRIDE;
        if constexpr (FMT == 1) {
            const float *sc = reinterpret_cast<const float *>(ring + RING_X + stage * SCB);
#pragma unroll
            for (int i = 0; i < FN; ++i) {
                const int r = wn * TN + i * 32 + fr;
                f.s[i] = sc[r];
                f.c[i] = sc[BN + r];
            }
        }
        if constexpr (W2) {
            const uint8_t *sw = ring + S * BM * 128 + ((kt >> 1) & 1) * (BN * 128);
#pragma unroll
            for (int i = 0; i < FN; ++i) {
                const int r = wn * TN + i * 32 + fr, c = (kt & 1) * 4 + 2 * kg + h;
                const uint4 v = *reinterpret_cast<const uint4 *>(sw + r * 128 + ((c ^ ((r >> 1) & 7)) * 16));
                f.w[0][i] = make_uint2(v.x, v.y);
                f.w[1][i] = make_uint2(v.z, v.w);
            }
#pragma unroll
            for (int kl = 0; kl < K16; ++kl)
#pragma unroll
                for (int j = 0; j < FM; ++j) {
                    const int r = wm * TM + j * 32 + fr, c = 4 * kg + 2 * h + kl;
                    f.x[kl][j] = *reinterpret_cast<const half8 *>(sx + r * 128 + ((c ^ ((r >> 1) & 7)) * 16));
                }
        } else {
            const uint8_t *sw = sx + BM * 128;
#pragma unroll
            for (int kl = 0; kl < K16; ++kl) {
                const int k16 = kg * K16 + kl;
#pragma unroll
                for (int i = 0; i < FN; ++i) {
                    const int r = wn * TN + i * 32 + fr;
                    f.w[kl][i] = *reinterpret_cast<const uint2 *>(sw + r * 64 + ((k16 ^ ((r >> 2) & 3)) * 16) + h * 8);
                }
#pragma unroll
                for (int j = 0; j < FM; ++j) {
                    const int r = wm * TM + j * 32 + fr, c = 2 * k16 + h;
                    f.x[kl][j] = *reinterpret_cast<const half8 *>(sx + r * 128 + ((c ^ ((r >> 1) & 7)) * 16));
                }
            }
        }
    };
    auto mma = [&](const Frag &f) {
#pragma unroll
        for (int kl = 0; kl < K16; ++kl) {
            half8 a[FN];
#pragma unroll
            for (int i = 0; i < FN; ++i) {
                if constexpr (FMT == 1) a[i] = u8x8_affine(f.w[kl][i], f.s[i], f.c[i]);
                else a[i] = i8x8_to_half8(f.w[kl][i]);
            }
#pragma unroll
            for (int i = 0; i < FN; ++i)
#pragma unroll
                for (int j = 0; j < FM; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], f.x[kl][j], acc[i][j], 0, 0, 0);
        }
    };
    // Wait until this wave's DMA for the step about to be read has landed
    // (the LATER steps after it may stay in flight), then let every wave see
    // every unit.  The barrier also orders every wave's reads of a stage
    // before the DMA that refills it.
    auto ready = [&](auto later) {
        wait_vmcnt<decltype(later)::value * NOUT>();
        __syncthreads();
    };
    using Ls2 = std::integral_constant<int, S - 2>;
    using Ls1 = std::integral_constant<int, S - 1>;

    if constexpr (W2) {
        // Iteration u (step kt = base + u): wait until step kt+1 has landed,
        // read its fragments while the MFMAs of kt run, then refill: odd
        // iterations first load the W pair (kt+3, kt+4) into the slot of the
        // pair (kt-1, kt), whose last fragments were read before this
        // iteration's barrier; every iteration loads X of step kt+4 into the
        // X stage of kt.  vmcnt counts (loads retire in order): an even
        // iteration needs everything through iteration u-3 (its W pair was the
        // first load there), so iterations u-2 (X) and u-1 (W, X) may stay in
        // flight; an odd one needs the W pair of iteration u-2, so that
        // iteration's X and iteration u-1's X may (the affine scales count
        // with their X stage).  The prologue issues steps 0-3 as iterations
        // -4..-1 would have.
        constexpr int WAIT_EVEN = 2 * XOPS + WUW, WAIT_ODD = 2 * XOPS;
        Frag f[2];
        dma(0, 0);
        dma_w(0, 0);
        dma(1, 1);
        dma(2, 2);
        dma_w(1, 2);
        dma(3, 3);
        wait_vmcnt<3 * XOPS + WUW>();
        __syncthreads();
        fetch(0, 0, f[0]);
#pragma unroll 1
        for (int kt = 0; kt < nk; kt += 4) {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                if (u % 2 == 0) wait_vmcnt<WAIT_EVEN>();
                else wait_vmcnt<WAIT_ODD>();
                __syncthreads();
                fetch((u + 1) % 4, kt + u + 1, f[(u + 1) % 2]);
                mma(f[u % 2]);
                if (u % 2 == 1) dma_w(((kt + u + 3) >> 1) & 1, kt + u + 3);
                dma(u, kt + u + 4);
            }
        }
    } else if constexpr (PINGPONG) {
        // Step k: step k+1 is ready, step k's stage is free (its fragments are
        // in registers), so DMA(k+S) refills it while the fragments of k+1
        // are read and the MFMAs of k run.
        constexpr int U = S % 2 == 0 ? S : 2 * S;
        Frag f[2];
#pragma unroll
        for (int j = 0; j < S; ++j) dma(j, j);
        ready(Ls1{});
        fetch(0, 0, f[0]);
#pragma unroll 1
        for (int kt = 0; kt < nk; kt += U) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                ready(Ls2{});
                if constexpr (KG == 2) {
                    // two k-groups: the step's MFMAs first, its DMA after them,
                    // so no wave queues behind the block's DMA burst before
                    // reaching its MFMAs (the ring leaves the DMA S - 1 steps
                    // to land): 1-3 % faster at 256x128 and 128x128, and at
                    // the two-wave groups of 128x64 and 64x64 (512x2048x5632
                    // 21.0 -> 19.8 us, 64x4096x4096 9.2 -> 8.6); 2 % slower
                    // with one group of 4 waves at 128x64
                    fetch((u + 1) % S, kt + u + 1, f[(u + 1) % 2]);
                    mma(f[u % 2]);
                    dma(u % S, kt + u + S);
                } else {
                    dma(u % S, kt + u + S);
                    fetch((u + 1) % S, kt + u + 1, f[(u + 1) % 2]);
                    mma(f[u % 2]);
                }
            }
        }
    } else {
        Frag f;
#pragma unroll
        for (int j = 0; j < S - 1; ++j) dma(j, j);
#pragma unroll 1
        for (int kt = 0; kt < nk; kt += S) {
#pragma unroll
            for (int u = 0; u < S; ++u) {
                ready(Ls2{});
                dma((u + S - 1) % S, kt + u + S - 1);
                fetch(u % S, kt + u, f);
                mma(f);
            }
        }
    }
    wait_vmcnt<0>();  // no DMA in flight past this point

    if constexpr (KG == 2) {
        // Group g finishes its half of the wave tile (see mine): it hands its
        // partial sums of the other tiles to the other group through the
        // (now idle) ring, lane-contiguous 16-byte pieces, and adds the other
        // group's partials of its own tiles.
        constexpr int HT = FN * FM / 2;  // tiles each group finishes
        static_assert(2 * WPG * HT * 16 * 64 * 4 <= RING, "exchange does not fit");
        float4 *xch = reinterpret_cast<float4 *>(&ring[0]);
        // index of tile (i, j) among the half it belongs to (the same in both groups)
        auto hidx = [&](int i, int j) { return KSPLIT_M ? i * (FM / 2) + j / 2 : (i / 2) * FM + j; };
        // slot of (target group, wave position, tile, quad r4), then lane
        auto slot = [&](int tg, int ti, int r4) { return ((tg * WPG + wq) * HT + ti) * 4 + r4; };
        __syncthreads();  // every wave is done with the ring
#pragma unroll
        for (int i = 0; i < FN; ++i)
#pragma unroll
            for (int j = 0; j < FM; ++j) {
                if (mine(i, j)) continue;
#pragma unroll
                for (int r4 = 0; r4 < 4; ++r4)
                    xch[slot(1 - kg, hidx(i, j), r4) * 64 + lane] =
                        make_float4(acc[i][j][4 * r4], acc[i][j][4 * r4 + 1], acc[i][j][4 * r4 + 2], acc[i][j][4 * r4 + 3]);
            }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < FN; ++i) {
#pragma unroll
            for (int j = 0; j < FM; ++j) {
                if (!mine(i, j)) continue;
#pragma unroll
                for (int r4 = 0; r4 < 4; ++r4) {
                    const float4 o = xch[slot(kg, hidx(i, j), r4) * 64 + lane];
                    acc[i][j][4 * r4] += o.x;
                    acc[i][j][4 * r4 + 1] += o.y;
                    acc[i][j][4 * r4 + 2] += o.z;
                    acc[i][j][4 * r4 + 3] += o.w;
                }
            }
        }
    }

    // Split-K: the tiles this wave finishes go to slot (tile, split) of the
    // workspace as lane-contiguous float4 pieces, stored and later read with
    // sc1 (device-coherent: the blocks of a tile may sit on different XCDs,
    // whose L2s are not coherent with each other).  Once its pieces have
    // landed, a block counts itself on the tile's counter; the block that
    // arrives last clears the counter for the next launch and adds all the
    // splits' partials in split order (deterministic whichever block is last)
    // before the epilogue.  No block waits for another.
    //
    // Ordering.  The counter is a relaxed agent-scope atomic; what orders the
    // partials around it is the gfx9.4+ memory model itself (the one LLVM's
    // AMDGPU backend implements for agent scope on multi-XCD parts):
    //  * an sc1 store is an agent-scope store: it writes through this XCD's
    //    L2, and its vmcnt decrement is the acknowledgement that it is visible
    //    at agent scope.  `s_waitcnt vmcnt(0)` (an asm statement with a memory
    //    clobber, so the compiler keeps every store above it) then the barrier
    //    make every thread's pieces visible before thread 0 issues the atomic;
    //  * the atomic executes at the memory side (agent scope), after those
    //    acknowledged stores;
    //  * the last block's partial loads are sc1 (agent-scope) loads: they miss
    //    this XCD's possibly stale L2 lines and read the coherent values.  They
    //    are issued only after thread 0's atomic has returned (its result is
    //    what `last` is computed from, published through LDS across a barrier,
    //    which also keeps the compiler from hoisting them).
    // An agent-scope release/acquire pair on the counter would add an L2
    // write-back (buffer_wbl2) and invalidate per block, which the sc1 stores
    // and loads make unnecessary: with the stores and loads themselves at agent
    // scope there are no other writes to publish and no stale lines to read.
    if constexpr (BM == 64 && BN == 64) {  // only the 64x64 grids split (see launch_tiled)
        if (splits > 1) {
            constexpr int FT = FNO * FMO;  // tiles this wave finishes
            const size_t slot_floats = (size_t)BM * BN;
            // finished tile (i, jj) of this wave, in (feature, token) order
            auto fidx = [&](int i, int jj) { return (i / FKG) * FMO + (KSPLIT_M ? jj / 2 : jj); };
            auto piece = [&](int i, int jj, int r4) {
                return (((wave * FT + fidx(i, jj)) * 4 + r4) * 64 + lane) * 16u;
            };
            {
                const auto rs = make_rsrc(skw + ((size_t)tile * splits + split) * slot_floats, (uint32_t)slot_floats * 4u);
#pragma unroll
                for (int i = 0; i < FN; ++i) {
#pragma unroll
                    for (int jj = 0; jj < FM; ++jj) {
                        if (!mine(i, jj)) continue;
#pragma unroll
                        for (int r4 = 0; r4 < 4; ++r4) {
                            // whole vectors: a bit_cast of an ext-vector element reads element 0
                            const floatx4 v = {acc[i][jj][4 * r4], acc[i][jj][4 * r4 + 1], acc[i][jj][4 * r4 + 2],
                                               acc[i][jj][4 * r4 + 3]};
                            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), rs, piece(i, jj, r4),
                                                                   0, 16);
                        }
                    }
                }
            }
            wait_vmcnt<0>();  // this thread's pieces have landed
            __shared__ int last;
            __syncthreads();  // ... and every thread's
            if (t == 0)
                last = __hip_atomic_fetch_add(&skc[tile * kSkCounterStride], 1, __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT) == splits - 1;
            __syncthreads();
            if (!last) return;
            if (t == 0) __hip_atomic_store(&skc[tile * kSkCounterStride], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
            for (int i = 0; i < FN; ++i)
#pragma unroll
                for (int jj = 0; jj < FM; ++jj)
#pragma unroll
                    for (int r = 0; r < 16; ++r) acc[i][jj][r] = 0.0f;
            // UNR splits per round trip (their pieces loaded together, ~64
            // VGPRs), added in split order
            constexpr int PIECES = FT * 4, UNR = PIECES >= 16 ? 1 : 16 / PIECES;
            auto rsrc_of = [&](int sp) {
                return make_rsrc(skw + ((size_t)tile * splits + sp) * slot_floats, (uint32_t)slot_floats * 4u);
            };
#pragma unroll 1
            for (int sp0 = 0; sp0 < splits; sp0 += UNR) {
                floatx4 v[UNR][PIECES];
#pragma unroll
                for (int u = 0; u < UNR; ++u) {
                    const auto rs = rsrc_of(min(sp0 + u, splits - 1));
                    // (piece index from fidx, not a running count: a count past
                    // the runtime-skipped tiles would index v dynamically)
#pragma unroll
                    for (int i = 0; i < FN; ++i)
#pragma unroll
                        for (int jj = 0; jj < FM; ++jj) {
                            if (!mine(i, jj)) continue;
#pragma unroll
                            for (int r4 = 0; r4 < 4; ++r4)
                                v[u][fidx(i, jj) * 4 + r4] = __builtin_bit_cast(
                                    floatx4, __builtin_amdgcn_raw_buffer_load_b128(rs, piece(i, jj, r4), 0, 16));
                        }
                }
#pragma unroll
                for (int u = 0; u < UNR; ++u) {
                    if (sp0 + u >= splits) break;
#pragma unroll
                    for (int i = 0; i < FN; ++i)
#pragma unroll
                        for (int jj = 0; jj < FM; ++jj) {
                            if (!mine(i, jj)) continue;
#pragma unroll
                            for (int r4 = 0; r4 < 4; ++r4)
#pragma unroll
                                for (int e = 0; e < 4; ++e) acc[i][jj][4 * r4 + e] += v[u][fidx(i, jj) * 4 + r4][e];
                        }
                }
            }
        }
    }

    // Epilogue: acc[i][j][r] = D[feature 8*(r/4) + 4*(lane/32) + r%4][token lane%32]
    // of tile (features n0 + wn*TN + 32 i, tokens m0 + wm*TM + 32 j).
    // Staged through the (idle) ring: the scaled tile goes to LDS row by row,
    // then every row leaves as 16-byte pieces, a full row segment per group of
    // lanes, with the non-temporal policy.  Writing straight from the MFMA
    // layout puts 8-byte pieces of 32 rows in every store instruction; staged,
    // 2048x4096x4096 took 70.9 -> 67.6 us, N = 11008 194.6 -> 182.5 us.
    // PAIR stages g and u as fp16 and leaves as h = silu(g) * u.
    auto staged = [&](auto eb_c) {
        constexpr int EB = decltype(eb_c)::value;  // staged element bytes
        constexpr int RS = BN * EB + 16;           // padded LDS row stride
        static_assert(BM * RS <= RING, "output staging does not fit in the ring");
        uint8_t *ot = reinterpret_cast<uint8_t *>(&ring[0]);
        __syncthreads();  // every wave is done with the ring (and the k-group exchange)
#pragma unroll
        for (int i = 0; i < FN; ++i) {
            if (!KSPLIT_M && !mine(i, 0)) continue;  // the other k-group finishes this tile
            const int io = i / FKG;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int fl = feat(io, g);  // feature within the tile
                const int wr = wrow(fl);     // its weight row (PAIR: of the gate or the up weight)
                float sc[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) sc[r] = wr + r < NL ? (FMT == 0 ? esc[io][g][r] : 1.0f) : 0.0f;
#pragma unroll
                for (int j = 0; j < FM; ++j) {
                    if (!mine(i, j)) continue;
                    uint8_t *dst = ot + (wm * TM + j * 32 + fr) * RS + fl * EB;
                    const float tf = tfac[j];
                    const float v0 = acc[i][j][4 * g] * sc[0] * tf, v1 = acc[i][j][4 * g + 1] * sc[1] * tf;
                    const float v2 = acc[i][j][4 * g + 2] * sc[2] * tf, v3 = acc[i][j][4 * g + 3] * sc[3] * tf;
                    if constexpr (EB == 2) {
                        const h2_t lo = {(_Float16)v0, (_Float16)v1}, hi = {(_Float16)v2, (_Float16)v3};
                        *reinterpret_cast<uint2 *>(dst) =
                            make_uint2(__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi));
                    } else {
                        *reinterpret_cast<float4 *>(dst) = make_float4(v0, v1, v2, v3);
                    }
                }
            }
        }
        __syncthreads();
        if constexpr (ROPE) {
            // 8 threads per tile row: thread c rotates the pairs (4c + e, 4c + e + 32)
            const int c = t % 8, hh = n0 / 64, kvh = hh - ro.n_heads;
            const bool rot = kvh < ro.n_kv;  // q and k heads; v is copied
#pragma unroll
            for (int ps = 0; ps < BM / RRP; ++ps) {
                const int row = ps * RRP + t / 8, sr = m0 + row;
                if (sr >= M) continue;
                const float4 a = *reinterpret_cast<const float4 *>(ot + row * RS + c * 16);
                const float4 b = *reinterpret_cast<const float4 *>(ot + row * RS + (c + 8) * 16);
                const float av[4] = {a.x, a.y, a.z, a.w}, bv[4] = {b.x, b.y, b.z, b.w};
                const float cs[8] = {rcs[ps][0].x, rcs[ps][0].y, rcs[ps][0].z, rcs[ps][0].w,
                                     rcs[ps][1].x, rcs[ps][1].y, rcs[ps][1].z, rcs[ps][1].w};
                h2_t lo[2], hi[2];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float cx = cs[2 * e], sy = cs[2 * e + 1];
                    lo[e / 2][e % 2] = (_Float16)(rot ? av[e] * cx - bv[e] * sy : av[e]);
                    hi[e / 2][e % 2] = (_Float16)(rot ? av[e] * sy + bv[e] * cx : bv[e]);
                }
                const int pos = ro.p0 + sr;
                _Float16 *dst = hh < ro.n_heads ? static_cast<_Float16 *>(Yv) + ((size_t)sr * ro.n_heads + hh) * 64
                                : rot ? ro.kc + ((size_t)kvh * ro.max_seq + pos) * 64
                                      : ro.vc + ((size_t)(kvh - ro.n_kv) * ro.max_seq + pos) * 64;
                *reinterpret_cast<uint2 *>(dst + 4 * c) =
                    make_uint2(__builtin_bit_cast(uint32_t, lo[0]), __builtin_bit_cast(uint32_t, lo[1]));
                *reinterpret_cast<uint2 *>(dst + 32 + 4 * c) =
                    make_uint2(__builtin_bit_cast(uint32_t, hi[0]), __builtin_bit_cast(uint32_t, hi[1]));
            }
            return;
        }
        constexpr int OB = PAIR ? HB * 2 : BN * EB;  // output bytes per tile row
        constexpr int CPR = OB / 16;                 // 16-byte pieces per tile row
        constexpr int RPP = 64 * NW / CPR;           // rows per pass
        static_assert(BM % RPP == 0, "copy-out passes");
        constexpr int OE = PAIR ? 2 : EB;            // output element bytes
        // rows past M fall outside the resource; pieces past the row are masked
        const auto ry = make_rsrc(static_cast<uint8_t *>(Yv) + ((size_t)m0 * NL + nw0) * OE,
                                  (uint32_t)min(BM, M - m0) * (uint32_t)NL * OE);
        const int c = t % CPR;
        const bool col_ok = nw0 + c * (16 / OE) < NL;
#pragma unroll
        for (int ps = 0; ps < BM / RPP; ++ps) {
            const int row = ps * RPP + t / CPR;
            uint4 v = *reinterpret_cast<const uint4 *>(ot + row * RS + c * 16);
            if constexpr (PAIR) {
                // silu(g) * u in f32 (v / (1 + e^-v), the reference's silu), rounded to fp16
                const half8 gv = __builtin_bit_cast(half8, v);
                const half8 uv = *reinterpret_cast<const half8 *>(ot + row * RS + HB * 2 + c * 16);
                half8 hv;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float gf = (float)gv[e];
                    hv[e] = (_Float16)(gf / (1.0f + expf(-gf)) * (float)uv[e]);
                }
                v = __builtin_bit_cast(uint4, hv);
            }
            const uint32_t off = col_ok ? (uint32_t)row * (uint32_t)NL * OE + (uint32_t)c * 16u : kOOB;
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), ry, off, 0, 2);
        }
    };
    if constexpr (ROPE) {
        staged(std::integral_constant<int, 4>{});  // f32 rows, rotated and written as fp16 q / k / v
        return;
    } else if constexpr (PAIR) {
        staged(std::integral_constant<int, 2>{});  // the host guarantees I % 8 == 0 and fp16 h
        return;
    } else {
        if ((y_f16 ? NL % 8 == 0 : NL % 4 == 0) && (int64_t)BM * NL * (y_f16 ? 2 : 4) < (1ll << 31)) {
            if (y_f16) staged(std::integral_constant<int, 2>{});
            else staged(std::integral_constant<int, 4>{});
            return;
        }
#pragma unroll
        for (int i = 0; i < FN; ++i) {
            if (!KSPLIT_M && !mine(i, 0)) continue;  // the other k-group finishes this tile
            const int io = i / FKG;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int nb = n0 + feat(io, g);  // weight row
                float sc[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) sc[r] = nb + r < N ? (FMT == 0 ? esc[io][g][r] : 1.0f) : 0.0f;
#pragma unroll
                for (int j = 0; j < FM; ++j) {
                    const int mm = m0 + wm * TM + j * 32 + fr;
                    if (!mine(i, j) || mm >= M) continue;
                    float v[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r) v[r] = acc[i][j][4 * g + r] * sc[r] * tfac[j];
                    const size_t o = (size_t)mm * N + nb;
                    if (nb + 4 <= N && (N % 4) == 0) {
                        if (y_f16) {
                            const h2_t lo = {(_Float16)v[0], (_Float16)v[1]}, hi = {(_Float16)v[2], (_Float16)v[3]};
                            *reinterpret_cast<uint2 *>(reinterpret_cast<_Float16 *>(Yv) + o) =
                                make_uint2(__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi));
                        } else {
                            *reinterpret_cast<float4 *>(reinterpret_cast<float *>(Yv) + o) =
                                make_float4(v[0], v[1], v[2], v[3]);
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
    }
}

// Split-K for 64x64 tile grids that leave CUs idle (few tokens: each block
// would otherwise walk all K alone, at a latency-bound rate per k-step): up
// to half the CUs, as many splits as keep one block per CU; up to 3/4, two
// splits (the 64x64 kernel fits three blocks per CU); at least 8 k-steps per
// split, within the context's workspace.  Measured at 4096x4096: 64 tiles
// 18.8 -> 10.3 us (4 splits; 8: 11.6), 128 tiles 18.6 -> 13.2 (2 splits),
// 192 tiles 18.6 -> 17.5 (2), 256 tiles best unsplit; 172 tiles at
// N = 11008: 19.0 -> 17.7 (2).  Only on the context's own stream (ws.partials
// is null otherwise); the larger tiles gained nothing from splitting (their
// LDS rings allow one block per CU).
// SwiGLU's up weight beside the gate weight of a PAIR launch (see
// k_gemm_rowwise); n_split = rows of each weight, 0: no pair.
struct GemmPair {
    const uint8_t *w = nullptr;
    const float *scales = nullptr;
    int64_t n_split = 0;
};

template <int BM, int BN, bool PINGPONG, int S, int NW, int WGN, int KG = 1, bool W2 = false, bool PAIR = false>
int launch_tiled(const rq_qweight &w, const float *scales, int fmt, const void *x, void *y, rq_dtype yt, int64_t m,
                 int gm, int64_t cus, const GemmWorkspace &ws, hipStream_t s, const GemmPair &pair = GemmPair{},
                 const RopeOut *rope = nullptr, const float *xscale = nullptr) {
    const int64_t N = w.n_out, K = w.k_in;
    const int tiles_m = (int)cdiv(m, BM), tiles_n = (int)cdiv(N, BN);
    const int64_t tiles = (int64_t)tiles_m * tiles_n;
    if (tiles > 0x7fffffff) return RQ_ERR_UNSUPPORTED;
    const int64_t nk = K / 64;
    int64_t splits = 1;
    if (BM == 64 && BN == 64 && !rope && ws.partials && nk >= 16 && 4 * tiles <= 3 * cus && tiles <= ws.n_counters) {
        splits = std::min<int64_t>(nk / 8, 2 * tiles <= cus ? cus / tiles : 2);
        while (splits > 1 && (size_t)(tiles * splits) * BM * BN > ws.floats) --splits;
        splits = cdiv(nk, cdiv(nk, splits));  // every split gets k-steps (the kernel's ks = ceil(nk / splits))
    }
    auto go = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, dim3((unsigned)(tiles * splits)), dim3(64 * NW), 0, s, (const uint8_t *)w.codes,
                           scales, (const _Float16 *)x, y, yt == RQ_F16 ? 1 : 0, (int)m, (int)N, (int)K, tiles_m,
                           tiles_n, gm < 1 ? 1 : gm, (int)splits, ws.partials, ws.counters, fmt == 1 ? w.group : 64,
                           pair.w, pair.scales, (int)(pair.n_split ? pair.n_split : N), rope ? *rope : RopeOut{},
                           xscale);
    };
    if constexpr (BN == 64 && !PAIR) {
        if (rope) {
            if (fmt == 1) go(k_gemm_rowwise<BM, BN, PINGPONG, S, NW, WGN, KG, W2, 1, false, true>);
            else go(k_gemm_rowwise<BM, BN, PINGPONG, S, NW, WGN, KG, W2, 0, false, true>);
            RQ_LAUNCH_CHECK();
            return RQ_OK;
        }
    }
    if constexpr (PAIR) {
        if (fmt == 1) go(k_gemm_rowwise<BM, BN, PINGPONG, S, NW, WGN, KG, W2, 1, true>);
        else go(k_gemm_rowwise<BM, BN, PINGPONG, S, NW, WGN, KG, W2, 0, true>);
    }
    else if (fmt == 1) go(k_gemm_rowwise<BM, BN, PINGPONG, S, NW, WGN, KG, W2, 1>);
    else go(k_gemm_rowwise<BM, BN, PINGPONG, S, NW, WGN, KG, W2, 0>);
    RQ_LAUNCH_CHECK();
    return RQ_OK;
}

// Input preparation (stream-ordered before the GEMM it feeds).
// Affine scales: out[g][0][n] = s[n][g], out[g][1][n] = b[n][g] - 1024 s[n][g]
// (gpr = groups per row; b NULL reads as 0), through 64 x 64 LDS tiles so
// both the reads along g and the writes along n are coalesced.
__global__ __launch_bounds__(256) void k_affine_prep(const float *__restrict__ s, const float *__restrict__ b, int N,
                                                     int gpr, float *__restrict__ out) {
    __shared__ float ts[64][65], tb[64][65];
    const int n0 = blockIdx.x * 64, g0 = blockIdx.y * 64, t = threadIdx.x;
    for (int i = t; i < 64 * 64; i += 256) {
        const int r = i / 64, c = i % 64, n = n0 + r, g = g0 + c;
        const bool ok = n < N && g < gpr;
        const size_t src = (size_t)n * gpr + g;
        ts[r][c] = ok ? s[src] : 0.0f;
        tb[r][c] = ok && b ? b[src] : 0.0f;
    }
    __syncthreads();
    for (int i = t; i < 64 * 64; i += 256) {
        const int r = i / 64, c = i % 64, g = g0 + r, n = n0 + c;
        if (g < gpr && n < N) {
            const float sv = ts[c][r];
            out[((size_t)g * 2) * N + n] = sv;
            out[((size_t)g * 2 + 1) * N + n] = __builtin_fmaf(-1024.0f, sv, tb[c][r]);
        }
    }
}

}  // namespace

// Size of the prepared scale table of an affine weight the GEMM serves
// (group a multiple of 64 dividing k_in, table addressable with 32-bit
// offsets), else 0.
size_t affine_prep_bytes(const rq_qweight &w) {
    if (w.format != RQ_Q_AFFINE_U8 || w.group <= 0 || w.group % 64 != 0 || w.k_in <= 0 || w.n_out <= 0 ||
        w.k_in % w.group != 0)
        return 0;
    const uint64_t b = (uint64_t)(w.k_in / w.group) * (uint64_t)w.n_out * 8u;
    return b > 0xffffffffull ? 0 : (size_t)b;
}

int launch_affine_prep(const rq_qweight &w, float *table, hipStream_t s) {
    const int64_t N = w.n_out, gpr = w.k_in / w.group;
    hipLaunchKernelGGL(k_affine_prep, dim3((unsigned)cdiv(N, 64), (unsigned)cdiv(gpr, 64)), dim3(256), 0, s, w.scales,
                       w.biases, (int)N, (int)gpr, table);
    RQ_LAUNCH_CHECK();
    return RQ_OK;
}

namespace {

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// f32 activation rows to fp16 (round to nearest even), one block per row: the
// row is scaled by the power of two 2^-e that puts its largest magnitude in
// [2^14, 2^15) and rs[row] = 2^e, which the GEMM's epilogue multiplies back
// (exact).  Any finite row fits fp16 that way, small rows keep fp16's full
// precision, and a row whose values all lie in fp16's normal range gives the
// same products as a plain conversion (scaling by a power of two commutes
// with rounding there).  K % 8 == 0.  NI > 0 (K <= NI * 2048): each thread
// holds its NI 8-value chunks in registers from the maximum to the
// conversion, so the row is read once; NI == 0 reads it twice (the second
// read hits L2).
template <int NI>
__global__ __launch_bounds__(256) void k_cast_f16_rows(const float *__restrict__ x, _Float16 *__restrict__ y,
                                                       float *__restrict__ rs, int K) {
    __shared__ float wmax[4];
    const size_t row = blockIdx.x;
    const float4 *xr = reinterpret_cast<const float4 *>(x + row * K);
    half8 *yr = reinterpret_cast<half8 *>(y + row * K);
    const int n8 = K / 8, t = threadIdx.x, lane = t & 63;
    auto amax8 = [](float4 a, float4 b) {
        return fmaxf(fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w))),
                     fmaxf(fmaxf(fabsf(b.x), fabsf(b.y)), fmaxf(fabsf(b.z), fabsf(b.w))));
    };
    float amax = 0.0f;
    float4 va[NI > 0 ? NI : 1], vb[NI > 0 ? NI : 1];
    if constexpr (NI > 0) {
#pragma unroll
        for (int j = 0; j < NI; ++j) {  // every load in flight before the first use
            const int i = t + 256 * j;
            va[j] = i < n8 ? xr[2 * i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            vb[j] = i < n8 ? xr[2 * i + 1] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
#pragma unroll
        for (int j = 0; j < NI; ++j) amax = fmaxf(amax, amax8(va[j], vb[j]));
    } else {
        for (int i = t; i < n8; i += 256) amax = fmaxf(amax, amax8(xr[2 * i], xr[2 * i + 1]));
    }
    amax = fmaxf(amax, dpp_f<0xB1>(amax));   // quad_perm [1,0,3,2]
    amax = fmaxf(amax, dpp_f<0x4E>(amax));   // quad_perm [2,3,0,1]
    amax = fmaxf(amax, dpp_f<0x141>(amax));  // row_half_mirror
    amax = fmaxf(amax, dpp_f<0x140>(amax));  // row_mirror: each 16-lane row holds its maximum
    const auto rl = [](float v, int l) {
        return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
    };
    amax = fmaxf(fmaxf(rl(amax, 0), rl(amax, 16)), fmaxf(rl(amax, 32), rl(amax, 48)));
    if (lane == 0) wmax[t >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    // amax = f * 2^E, f in [0.5, 1); a zero, infinite or NaN maximum gives
    // E = 0 (an inf or NaN stays one)
    const int e = max(__builtin_amdgcn_frexp_expf(amax) - 15, -126);
    auto cvt = [e](float4 a, float4 b) {
        return half8{(_Float16)__builtin_amdgcn_ldexpf(a.x, -e), (_Float16)__builtin_amdgcn_ldexpf(a.y, -e),
                     (_Float16)__builtin_amdgcn_ldexpf(a.z, -e), (_Float16)__builtin_amdgcn_ldexpf(a.w, -e),
                     (_Float16)__builtin_amdgcn_ldexpf(b.x, -e), (_Float16)__builtin_amdgcn_ldexpf(b.y, -e),
                     (_Float16)__builtin_amdgcn_ldexpf(b.z, -e), (_Float16)__builtin_amdgcn_ldexpf(b.w, -e)};
    };
    if constexpr (NI > 0) {
#pragma unroll
        for (int j = 0; j < NI; ++j) {
            const int i = t + 256 * j;
            if (i < n8) yr[i] = cvt(va[j], vb[j]);
        }
    } else {
        for (int i = t; i < n8; i += 256) yr[i] = cvt(xr[2 * i], xr[2 * i + 1]);
    }
    if (t == 0) rs[row] = __builtin_amdgcn_ldexpf(1.0f, e);
}

// Whether a grid of bm x bn tiles over m x N still has >= 2/3 as many tiles as
// the device has CUs (and the tile is not taller than the tokens, rounded up
// to 64): the tile choice below.
bool tile_fills(int64_t m, int64_t N, int64_t cus, int bm, int bn) {
    return bm <= std::max<int64_t>(64, m) && cdiv(m, bm) * cdiv(N, bn) * 3 >= 2 * cus;
}

// The fp16-activation GEMM over m rows, tile chosen by shape.
int gemm_tiles(const rq_qweight &w, const float *scales, int fmt, const void *x, void *y, rq_dtype yt, int64_t m,
               int64_t cus, const GemmWorkspace &ws, hipStream_t s, const GemmPair &pair = GemmPair{},
               const float *xscale = nullptr) {
    const int64_t N = w.n_out;
    // The largest tile whose grid still has >= 2/3 as many tiles as the device
    // has CUs: a block streams its X and W panels through one CU at a latency-
    // bound rate, so a grid that leaves CUs idle loses more than smaller tiles
    // cost.  Measured (N = K = 4096): m = 256 64x64 19.9 us (128x128: 36.2),
    // m = 512 128x64 28.1 us (38.4), m = 768 128x128 39.0, m = 1536 256x128
    // 61.2 us (128x128: 76.3); N = 11008, m = 256: 128x128 39.1 (64x64: 41.1).
    // Groups of 4 token panels per XCD and the ping-pong fragments beat
    // token-major order and single buffering by 5-15 % at m = 2048.  The two
    // large tiles run two k-groups of 4 waves with the weight staged in pairs
    // of k-steps; 128x64 and 64x64 two k-groups of 2 waves, each wave all the
    // tile's tokens (two groups of 4 waves there, each wave still expanding
    // its W fragment for 1-2 MFMAs, measured 2-4 % slower than one group of 4
    // and than these).  128x256 rather than 256x128: for the same outputs per block
    // (one 128x64 wave tile per wave) it stages 32 KiB per k-step instead of
    // 40, in 256 cache lines instead of 320 (2048x4096x4096 64.5 -> 62.1 us,
    // N = 11008 176.4 -> 171.2, K = 11008 162.5 -> 156.9 us in one run), and
    // it fills the device whenever 256x128 would.
    // a tile taller than the tokens (rounded up to 64) only multiplies padding:
    // 64 x 11008 x 4096 took 23.6 us on 128x64 tiles, 17.7 on split 64x64 ones
    auto fills = [&](int bm, int bn) { return tile_fills(m, N, cus, bm, bn); };
    if (pair.n_split) {  // gate and up: the two large tiles only (the caller falls back otherwise)
        if (fills(128, 256))
            return launch_tiled<128, 256, true, 4, 8, 4, 2, true, true>(w, scales, fmt, x, y, yt, m, 4, cus, ws, s, pair);
        if (fills(128, 128))
            return launch_tiled<128, 128, true, 4, 8, 2, 2, true, true>(w, scales, fmt, x, y, yt, m, 4, cus, ws, s, pair);
        return RQ_ERR_UNSUPPORTED;
    }
    const GemmPair np{};
    if (fills(128, 256))
        return launch_tiled<128, 256, true, 4, 8, 4, 2, true>(w, scales, fmt, x, y, yt, m, 4, cus, ws, s, np, nullptr,
                                                              xscale);
    if (fills(128, 128))
        return launch_tiled<128, 128, true, 4, 8, 2, 2, true>(w, scales, fmt, x, y, yt, m, 4, cus, ws, s, np, nullptr,
                                                              xscale);
    if (fills(128, 64))
        return launch_tiled<128, 64, true, 6, 4, 2, 2>(w, scales, fmt, x, y, yt, m, 4, cus, ws, s, np, nullptr, xscale);
    return launch_tiled<64, 64, true, 4, 4, 2, 2>(w, scales, fmt, x, y, yt, m, 4, cus, ws, s, np, nullptr, xscale);
}

}  // namespace

// Returns RQ_ERR_UNSUPPORTED (without launching) outside what k_gemm_rowwise
// serves; the caller then uses the generic kernel.  Per-row int8 weights with
// fp16 activations run directly.  Affine weights (group a multiple of 64
// dividing k_in) and f32 activations are first prepared in the workspace's
// preparation area (context stream only): the scales transposed to
// [group][row] and/or the activations cast to fp16, a chunk of rows at a time
// when they do not fit, each chunk then multiplied by the same kernel.
// SwiGLU's gate and up in one launch with the silu*mul epilogue:
// h = fp16(silu(g) * u), g = fp16(X . deq(gate)^T), u = fp16(X . deq(up)^T),
// h fp16 [m][I].  The two weights form one grid of 2 I rows, each tile taking
// the same rows of both, so the tile heuristic sees the combined width (at 512
// tokens x 5632 features: 128x256 tiles over both instead of two launches of
// 128x128 tiles that each leave a third of the CUs idle) and g and u never
// leave the block.  Weights of one shape, per-row int8 or affine u8 with
// their load-time tables (rq_qweight_prepare, the same group), fp16
// activations, I % 8 == 0; RQ_ERR_UNSUPPORTED otherwise, or when the grid is
// too small for the two large tiles.
// A Llama layer's packed q/k/v projection with the rotary epilogue (see
// k_gemm_rowwise, ROPE): q fp16 [m][n_heads][64] to q, k and v into the
// caches at positions ro.p0 .. ro.p0 + m - 1.  Weights of (n_heads + 2 n_kv)
// 64 rows, per-row int8 or affine u8 with the load-time table
// (rq_qweight_prepare), fp16 x, and a token count whose tile choice is 64
// wide (64x64 or 128x64); RQ_ERR_UNSUPPORTED (nothing launched) otherwise,
// and the caller runs the product and the rotation separately.
int launch_gemm_qkv_rope(const rq_qweight &w, const _Float16 *x, int64_t m, const RopeOut &ro, _Float16 *q,
                         int num_cus, const GemmWorkspace &ws, hipStream_t s) {
    const int64_t N = w.n_out, K = w.k_in;
    const bool affine = w.format == RQ_Q_AFFINE_U8;
    if (affine && !(w.prep && affine_prep_bytes(w) > 0)) return RQ_ERR_UNSUPPORTED;
    if ((!affine && w.format != RQ_Q_ROWWISE_I8) || K % 64 != 0 || K > (1 << 21) || m < 1 || m > 0x7fffffff ||
        N != (int64_t)(ro.n_heads + 2 * ro.n_kv) * 64 || !ro.rope || !ro.kc || !ro.vc || !aligned(w.codes, 16) ||
        !aligned(x, 16) || !aligned(q, 8) || !aligned(ro.kc, 8) || !aligned(ro.vc, 8) || !aligned(ro.rope, 16) ||
        (int64_t)ro.p0 + m > ro.max_seq)
        return RQ_ERR_UNSUPPORTED;
    const int64_t cus = num_cus > 0 ? num_cus : 256;
    if (tile_fills(m, N, cus, 128, 256) || tile_fills(m, N, cus, 128, 128)) return RQ_ERR_UNSUPPORTED;
    const float *sc = affine ? w.prep : w.scales;
    const int fmt = affine ? 1 : 0;
    if (tile_fills(m, N, cus, 128, 64))
        return launch_tiled<128, 64, true, 6, 4, 2, 2>(w, sc, fmt, x, q, RQ_F16, m, 4, cus, ws, s, GemmPair{}, &ro);
    return launch_tiled<64, 64, true, 4, 4, 2, 2>(w, sc, fmt, x, q, RQ_F16, m, 4, cus, ws, s, GemmPair{}, &ro);
}

int launch_gemm_swiglu(const rq_qweight &gate, const rq_qweight &up, const void *x, rq_dtype xt, void *h, int64_t m,
                       int num_cus, const GemmWorkspace &ws, hipStream_t s) {
    const int64_t I = gate.n_out, K = gate.k_in;
    // affine codes: both weights with their load-time tables (rq_qweight_prepare), the same group
    const bool affine = gate.format == RQ_Q_AFFINE_U8;
    if (affine && (up.format != RQ_Q_AFFINE_U8 || up.group != gate.group || !gate.prep || !up.prep ||
                   affine_prep_bytes(gate) == 0 || affine_prep_bytes(up) == 0))
        return RQ_ERR_UNSUPPORTED;
    if ((!affine && (gate.format != RQ_Q_ROWWISE_I8 || up.format != RQ_Q_ROWWISE_I8)) || up.n_out != I || up.k_in != K ||
        xt != RQ_F16 || I % 8 != 0 || K % 64 != 0 || K > (1 << 21) || !aligned(gate.codes, 16) ||
        !aligned(up.codes, 16) || !aligned(x, 16) || !aligned(h, 16) || m > 0x7fffffff || 2 * I > 0x7fffffff ||
        128 * I * 2 >= (1ll << 31))
        return RQ_ERR_UNSUPPORTED;
    rq_qweight w = gate;
    w.n_out = 2 * I;
    GemmPair pair;
    pair.w = static_cast<const uint8_t *>(up.codes);
    pair.scales = affine ? up.prep : up.scales;
    pair.n_split = I;
    return gemm_tiles(w, affine ? gate.prep : gate.scales, affine ? 1 : 0, x, h, RQ_F16, m, num_cus > 0 ? num_cus : 256,
                      ws, s, pair);
}

// Per-row int8 weight, fp16 activation rows each carrying the power of two
// xscale[row] (the epilogue multiplies it back): the matrix-core input
// gradient's GEMM (backward.hip).  RQ_ERR_UNSUPPORTED outside the tiles.
int launch_gemm_f16_scaled(const rq_qweight &w, const float *scales, const _Float16 *x, const float *xscale,
                           void *y, rq_dtype yt, int64_t m, int num_cus, const GemmWorkspace &ws, hipStream_t s) {
    const int64_t N = w.n_out, K = w.k_in;
    if (w.format != RQ_Q_ROWWISE_I8 || K % 64 != 0 || K > (1 << 21) || !aligned(w.codes, 16) || m > 0x7fffffff ||
        N > 0x7fffffff || !aligned(x, 16) || (yt == RQ_F16 ? !aligned(y, 8) : !aligned(y, 16)))
        return RQ_ERR_UNSUPPORTED;
    return gemm_tiles(w, scales, 0, x, y, yt, m, num_cus > 0 ? num_cus : 256, ws, s, GemmPair{}, xscale);
}

int launch_gemm(const rq_qweight &w, const void *x, rq_dtype xt, void *y, rq_dtype yt, int64_t m, int num_cus,
                const GemmWorkspace &ws, hipStream_t s) {
    const int64_t N = w.n_out, K = w.k_in;
    const int fmt = w.format == RQ_Q_AFFINE_U8 ? 1 : 0;
    // 32-bit buffer offsets: a 256-row panel of X (256 * K * 2 bytes) must stay below 2^31.
    if (K % 64 != 0 || K > (1 << 21) || !aligned(w.codes, 16) || m > 0x7fffffff || N > 0x7fffffff)
        return RQ_ERR_UNSUPPORTED;
    if (fmt == 1 && (w.group % 64 != 0 || K % w.group != 0)) return RQ_ERR_UNSUPPORTED;
    if (yt == RQ_F16 ? !aligned(y, 8) : !aligned(y, 16)) return RQ_ERR_UNSUPPORTED;
    if (!aligned(x, 16)) return RQ_ERR_UNSUPPORTED;
    const int64_t cus = num_cus > 0 ? num_cus : 256;
    if (fmt == 0 && xt == RQ_F16) return gemm_tiles(w, w.scales, 0, x, y, yt, m, cus, ws, s);
    // affine scales: the table prepared at load, else built here per call
    const bool table = fmt == 1 && w.prep && affine_prep_bytes(w) > 0;
    if (fmt == 1 && table && xt == RQ_F16) return gemm_tiles(w, w.prep, 1, x, y, yt, m, cus, ws, s);
    if (!ws.prep) return RQ_ERR_UNSUPPORTED;
    uint8_t *prep = static_cast<uint8_t *>(ws.prep);
    size_t used = 0;
    const float *scales = fmt == 1 && table ? w.prep : w.scales;
    if (fmt == 1 && !table) {
        const size_t sc_bytes = (affine_prep_bytes(w) + 255) & ~size_t(255);
        if (sc_bytes == 0 || sc_bytes > ws.prep_bytes / 2) return RQ_ERR_UNSUPPORTED;
        float *sct = reinterpret_cast<float *>(prep);
        const int st = launch_affine_prep(w, sct, s);
        if (st != RQ_OK) return st;
        scales = sct;
        used = sc_bytes;
    }
    if (xt == RQ_F16) return gemm_tiles(w, scales, fmt, x, y, yt, m, cus, ws, s);
    // f32 activations: cast a chunk of rows (a multiple of 128) to fp16, each
    // row scaled by a power of two (the factors after the rows), multiply it
    const size_t row_bytes = (size_t)K * 2 + 4;
    const int64_t chunk = std::min<int64_t>(m, (int64_t)((ws.prep_bytes - used - 256) / row_bytes) / 128 * 128);
    if (chunk < std::min<int64_t>(m, 128)) return RQ_ERR_UNSUPPORTED;
    _Float16 *x16 = reinterpret_cast<_Float16 *>(prep + used);
    float *xs = reinterpret_cast<float *>(prep + used + (((size_t)chunk * K * 2 + 255) & ~size_t(255)));
    const size_t eb = yt == RQ_F16 ? 2 : 4;
    for (int64_t r0 = 0; r0 < m; r0 += chunk) {
        const int64_t mc = std::min(chunk, m - r0);
        const float *xc = static_cast<const float *>(x) + r0 * K;
        const int64_t per = cdiv(K / 8, 256);  // 8-value chunks per thread
        if (per <= 1) hipLaunchKernelGGL(k_cast_f16_rows<1>, dim3((unsigned)mc), dim3(256), 0, s, xc, x16, xs, (int)K);
        else if (per <= 2) hipLaunchKernelGGL(k_cast_f16_rows<2>, dim3((unsigned)mc), dim3(256), 0, s, xc, x16, xs, (int)K);
        else if (per <= 4) hipLaunchKernelGGL(k_cast_f16_rows<4>, dim3((unsigned)mc), dim3(256), 0, s, xc, x16, xs, (int)K);
        else if (per <= 8) hipLaunchKernelGGL(k_cast_f16_rows<8>, dim3((unsigned)mc), dim3(256), 0, s, xc, x16, xs, (int)K);
        else hipLaunchKernelGGL(k_cast_f16_rows<0>, dim3((unsigned)mc), dim3(256), 0, s, xc, x16, xs, (int)K);
        RQ_LAUNCH_CHECK();
        const int st = gemm_tiles(w, scales, fmt, x16, static_cast<uint8_t *>(y) + (size_t)r0 * (size_t)N * eb, yt, mc,
                                  cus, ws, s, GemmPair{}, xs);
        if (st != RQ_OK) return st;
    }
    return RQ_OK;
}

}  // namespace rq
