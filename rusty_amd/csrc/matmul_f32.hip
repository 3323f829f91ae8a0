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
#include "lds_dma.hpp"

namespace rq {
namespace {

constexpr int BM = 64, BN = 64, BK = 16, TH = 256;

// Operand loads without branches or selects on the loaded value: an
// out-of-range element loads element 0 (the callers never load from an empty
// operand) and is replaced by zero only when it is staged, after the loads of
// a whole step are in flight.  A branch around each load made the compiler
// wait for every load at its join (s_waitcnt vmcnt(0) per element), and a
// select right after the load waits for it just the same.
// logical A[r, c] with r < m, c < k; A stored [k, m] for MM_ATB
template <int V>
__device__ __forceinline__ bool in_a(int64_t r, int64_t c, int64_t m, int64_t k) { return r < m && c < k; }
template <int V>
__device__ __forceinline__ float raw_a(const float *a, int64_t r, int64_t c, int64_t m, int64_t k) {
    return a[in_a<V>(r, c, m, k) ? (V == MM_ATB ? c * m + r : r * k + c) : 0];
}
// logical B[r, c] with r < k, c < n; B stored [n, k] for MM_ABT
template <int V>
__device__ __forceinline__ bool in_b(int64_t r, int64_t c, int64_t k, int64_t n) { return r < k && c < n; }
template <int V>
__device__ __forceinline__ float raw_b(const float *b, int64_t r, int64_t c, int64_t k, int64_t n) {
    return b[in_b<V>(r, c, k, n) ? (V == MM_ABT ? c * k + r : r * n + c) : 0];
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

    // A tile BM x BK and B tile BK x BN, each thread's 4 + 4 elements coalesced
    // along the operand's contiguous dimension; the next step's elements are
    // loaded into registers before the current step's fmas run (all of them
    // in flight at once: stored to LDS one by one as they arrived, each load
    // had waited for the previous one).
    float ra[4], rb[4];
    auto a_at = [&](int i, int &r, int &c) {
        if constexpr (V == MM_ATB) { r = t % 64; c = t / 64 + 4 * i; }
        else { c = t % 16; r = t / 16 + 16 * i; }
    };
    auto b_at = [&](int i, int &r, int &c) {  // r: k within the step, c: column
        if constexpr (V == MM_ABT) { r = t % 16; c = t / 16 + 16 * i; }
        else { c = t % 64; r = t / 64 + 4 * i; }
    };
    auto load = [&](int64_t k0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            int r, c;
            a_at(i, r, c);
            ra[i] = raw_a<V>(a, m0 + r, k0 + c, m, k);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            int r, c;
            b_at(i, r, c);
            rb[i] = raw_b<V>(b, k0 + r, n0 + c, k, n);
        }
    };
    if (k > 0) load(0);
    for (int64_t k0 = 0; k0 < k; k0 += BK) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            int r, c;
            a_at(i, r, c);
            As[c][r] = in_a<V>(m0 + r, k0 + c, m, k) ? ra[i] : 0.0f;
            b_at(i, r, c);
            Bs[r][c] = in_b<V>(k0 + r, n0 + c, k, n) ? rb[i] : 0.0f;
        }
        __syncthreads();
        if (k0 + BK < k) load(k0 + BK);
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
            const int64_t r = m0 + ty + 16 * i, c = n0 + tx + 16 * j;
            if (r < m && c < n) out[r * n + c] = acc[i][j];
        }
}

// Grids of few 64x64 tiles (few rows or few columns: configs[0]'s 8 x 1024,
// a LoRA adapter's x . A with 16 columns) leave most CUs idle while each
// block walks all of k alone, 16 k-steps per pair of barriers.  There, a
// block owns a TR x TC output tile, one output per thread (TR * TC = 256),
// and the same k-ascending fma chain per output runs over k-chunks of KC
// staged in LDS by all the block's threads (coalesced along the operand's
// contiguous dimension); the next chunk's loads are in registers before the
// current chunk's chains run.  A is staged [TR][KC + 4] and B transposed,
// [TC][KC + 4] (16-byte rows: four k-steps of each operand per LDS read).
//
// The chunk loads are buffer loads at one per-thread 32-bit offset per
// operand plus a per-element stride held in scalar registers, with no bounds
// test: a position past the operand reads as zero (the buffer's size), and
// one past a row's end lands on a value of a row or column whose output is
// never stored, or on k past K, which no chain reads (a partial chunk's
// chains stop at K).  Per-element 64-bit addresses with clamped indices kept
// some 130 VGPRs live across the chunk loop, and the compiler moved the
// arriving values into AGPRs before the chains -- a wait for the loads it
// had just issued, so every chunk paid a memory round trip (1 x 4096 x 16:
// 45 us).  The host keeps every offset below 2^32 (chain_fits).  Waves whose
// rows all lie past m skip the chains (m = 1 with 16 rows per block: 3 of 4).
__device__ __forceinline__ float bload(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0));
}

template <int TC>
constexpr int chain_kc() { return TC == 16 || TC == 32 ? 512 : 256; }  // 64-80 KiB of LDS per chunk

// AH: A holds fp16 values (MM_AB only), loaded as 2-byte elements and
// widened exactly when staged -- the f32 matmul of the widened copy, without
// the copy (a LoRA adapter's x . A on fp16 activations).
template <int V, int TC, bool AH = false>
__global__ __launch_bounds__(TH) void k_matmul_f32_chain(const void *__restrict__ a, const float *__restrict__ b,
                                                         float *__restrict__ out, int64_t m, int64_t k, int64_t n) {
    static_assert(!AH || V == MM_AB, "fp16 A: C = A.B only");
    constexpr uint32_t EA = AH ? 2u : 4u;  // bytes per A element
    constexpr int TR = TH / TC;
    constexpr int KC = chain_kc<TC>();
    constexpr int P = KC / TH;                       // chunk rows of TH elements per contiguous row piece
    constexpr int AS = KC + 4;                       // padded A row (floats)
    constexpr int NA = TR * KC / TH, NB = KC * TC / TH;  // chunk elements per thread
    constexpr int G = 32;                            // k-steps per register set of the chains
    // (+ G: the chains' reads one register set past the chunk stay inside the arrays)
    __shared__ __attribute__((aligned(16))) float As[TR * AS + G];
    __shared__ __attribute__((aligned(16))) float Bs[TC * AS + G];
    const int t = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(t / 64);
    const int64_t r0 = (int64_t)blockIdx.y * TR, c0 = (int64_t)blockIdx.x * TC;
    const int tr = t / TC, tc = t % TC;  // this thread's output
    const uint32_t K = (uint32_t)k, M = (uint32_t)m, N = (uint32_t)n;
    const auto ra_ = make_rsrc(a, (uint32_t)(m * k * EA)), rb_ = make_rsrc(b, (uint32_t)(k * n * 4));
    // Element e of this thread in a chunk: LDS index and byte offset from the
    // thread's base offset (uniform per e); the bases advance by a chunk.
    //  A [m, k] (A [k, m] for MM_ATB), B [k, n] (B [n, k] for MM_ABT).
    uint32_t va, vb, da, db;
    if constexpr (V == MM_ATB) {
        va = ((uint32_t)(t / TR) * M + (uint32_t)r0 + (uint32_t)(t % TR)) * 4u;
        da = (uint32_t)KC * M * 4u;
    } else {
        va = ((uint32_t)r0 * K + (uint32_t)t) * EA;
        da = (uint32_t)KC * EA;
    }
    if constexpr (V == MM_ABT) {
        vb = ((uint32_t)c0 * K + (uint32_t)t) * 4u;
        db = (uint32_t)KC * 4u;
    } else {
        vb = ((uint32_t)(t / TC) * N + (uint32_t)c0 + (uint32_t)(t % TC)) * 4u;
        db = (uint32_t)KC * N * 4u;
    }
    auto a_soff = [&](int e) -> uint32_t {
        if constexpr (V == MM_ATB) return (uint32_t)(TC * e) * M * 4u;
        else return (uint32_t)(e / P) * K * EA + (uint32_t)(e % P) * (TH * EA);
    };
    auto a_lds = [&](int e) {
        if constexpr (V == MM_ATB) return (t % TR) * AS + t / TR + TC * e;
        else return (e / P) * AS + t + TH * (e % P);
    };
    auto b_soff = [&](int e) -> uint32_t {
        if constexpr (V == MM_ABT) return (uint32_t)(e / P) * K * 4u + (uint32_t)(e % P) * (TH * 4u);
        else return (uint32_t)(TR * e) * N * 4u;
    };
    auto b_lds = [&](int e) {
        if constexpr (V == MM_ABT) return (e / P) * AS + t + TH * (e % P);
        else return (t % TC) * AS + t / TC + TR * e;
    };
    float ra[NA], rb[NB];  // AH: ra holds the raw fp16 bits
    auto load = [&]() {
#pragma unroll
        for (int e = 0; e < NA; ++e) {
            if constexpr (AH)
                ra[e] = __builtin_bit_cast(float, (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(ra_, va, a_soff(e), 0));
            else
                ra[e] = bload(ra_, va, a_soff(e));
        }
#pragma unroll
        for (int e = 0; e < NB; ++e) rb[e] = bload(rb_, vb, b_soff(e));
        va += da;
        vb += db;
    };
    auto stage = [&]() {
#pragma unroll
        for (int e = 0; e < NA; ++e) {
            if constexpr (AH)
                As[a_lds(e)] = (float)__builtin_bit_cast(_Float16, (uint16_t)__builtin_bit_cast(uint32_t, ra[e]));
            else
                As[a_lds(e)] = ra[e];
        }
#pragma unroll
        for (int e = 0; e < NB; ++e) Bs[b_lds(e)] = rb[e];
    };
    // this wave's rows: (64 / TC) from 64 wave / TC
    const bool idle = r0 + 64 * wave / TC >= m;
    float acc = 0.0f;
    if (k > 0) load();
    for (int64_t k0 = 0; k0 < k; k0 += KC) {
        stage();
        __syncthreads();
        if (k0 + KC < k) load();  // in flight while this chunk's chains run
        const float *ar = As + tr * AS, *bc = Bs + tc * AS;
        if (idle) {
        } else if (k0 + KC <= k) {
            // two named register sets of G k-steps: the next set's LDS reads are
            // issued (unconditionally) before the current set's fmas (a
            // scheduling barrier keeps the compiler from sinking them below)
            float xa0[G], xb0[G], xa1[G], xb1[G];
            auto rd = [&](float *xa, float *xb, int kk) {
#pragma unroll
                for (int i = 0; i < G; i += 4) {
                    const float4 v = *reinterpret_cast<const float4 *>(ar + kk + i);
                    const float4 u = *reinterpret_cast<const float4 *>(bc + kk + i);
                    xa[i] = v.x;
                    xa[i + 1] = v.y;
                    xa[i + 2] = v.z;
                    xa[i + 3] = v.w;
                    xb[i] = u.x;
                    xb[i + 1] = u.y;
                    xb[i + 2] = u.z;
                    xb[i + 3] = u.w;
                }
            };
            auto fm = [&](const float *xa, const float *xb) {
#pragma unroll
                for (int i = 0; i < G; ++i) acc = __builtin_fmaf(xa[i], xb[i], acc);
            };
            rd(xa0, xb0, 0);
            for (int kk = 0; kk < KC; kk += 2 * G) {
                rd(xa1, xb1, kk + G);
                __builtin_amdgcn_sched_barrier(0);
                fm(xa0, xb0);
                rd(xa0, xb0, kk + 2 * G);  // at the chunk's end: read, not used
                __builtin_amdgcn_sched_barrier(0);
                fm(xa1, xb1);
            }
        } else {
            const int kc = (int)(k - k0);
            for (int kk = 0; kk < kc; ++kk) acc = __builtin_fmaf(ar[kk], bc[kk], acc);
        }
        __syncthreads();  // every chain is done with the chunk before it is overwritten
    }
    const int64_t r = r0 + tr, c = c0 + tc;
    if (r < m && c < n) out[r * n + c] = acc;
}

// The same chains fed through an LDS ring of NS chunks of KC = 256 k-steps
// filled by global -> LDS DMA (16 bytes per lane, no registers held), so
// NS - 1 chunks are in flight while one is multiplied.  A chain advances one
// dependent fma per 8.4 cycles (MI355X, one wave), 0.9 us per chunk, while a
// chunk's loads take about two: with one chunk in flight (the register-
// staged kernel above) every chunk waited for its data.  Each operand keeps
// its stored layout in LDS, as the DMA writes lane pieces contiguously:
//  * rows along k (A of MM_AB and MM_ABT, B of MM_ABT): [R][KC + 4], each
//    row's chunk one 1 KiB DMA unit; the chain reads four k-steps per ds_read_b128;
//  * rows along the outputs (A of MM_ATB, B of MM_AB and MM_ATB): [KC][C],
//    C = TR or TC columns, a unit covering 256 / C k-rows; the chain reads
//    one k-step per element (paired into ds_read2_b32).
// Units of a chunk: TR for A, TC for B, wave w issuing units w, w + 4, ...
// Positions past an operand read as zero or land in rows, columns or k that
// no stored output uses (as above); the dummy DMAs of chunks past K use an
// offset beyond every resource (operands < 2 GiB, chain_fits).  Requires
// 16-byte aligned operands and row pitches (ring_ok).
constexpr int RKC = 256;
constexpr uint32_t kOOBf = 0x80000000u;  // past every operand resource (operands < 2 GiB)
template <int V, int TC>
struct RingShape {
    static constexpr int TR = TH / TC;
    static constexpr bool AK = V != MM_ATB;  // A stored with rows along k
    static constexpr bool BK = V == MM_ABT;  // B stored with rows along k
    static constexpr int SA = AK ? TR * (RKC + 4) : RKC * TR;  // floats per stage
    static constexpr int SB = BK ? TC * (RKC + 4) : RKC * TC;
    static constexpr int ST = SA + SB;
    static constexpr int NS = 4 * ST * 4 <= 140 * 1024 ? 4 : 3;
    static constexpr int OPS = (TR + TC) / 4;  // DMA units per wave per chunk
    static_assert(3 * ST * 4 <= 140 * 1024 && (TR + TC) % 4 == 0, "ring does not fit");
};

template <int V, int TC>
__global__ __launch_bounds__(TH) void k_matmul_f32_ring(const float *__restrict__ a, const float *__restrict__ b,
                                                        float *__restrict__ out, int64_t m, int64_t k, int64_t n) {
    using RS = RingShape<V, TC>;
    constexpr int TR = RS::TR, NS = RS::NS, OPS = RS::OPS, SA = RS::SA, ST = RS::ST, AS = RKC + 4;
    constexpr int G = 32;
    // (+ G: the chains' reads one register set past a chunk stay inside the ring)
    __shared__ __attribute__((aligned(1024))) float ring[NS * ST + G * (TR + TC)];
    const int t = threadIdx.x, lane = t % 64;
    const int wave = __builtin_amdgcn_readfirstlane(t / 64);
    const int64_t r0 = (int64_t)blockIdx.y * TR, c0 = (int64_t)blockIdx.x * TC;
    const int tr = t / TC, tc = t % TC;
    const uint32_t K = (uint32_t)k, M = (uint32_t)m, N = (uint32_t)n;
    const auto rsa = make_rsrc(a, (uint32_t)(m * k * 4)), rsb = make_rsrc(b, (uint32_t)(k * n * 4));
    const uint32_t ring0 = lds_addr(&ring[0]);
    const int nck = (int)((k + RKC - 1) / RKC);

    // Byte offset of this lane's piece of unit i of chunk c (see above):
    // rows along k: row i of the panel, k = c KC + 4 lane; rows along the
    // outputs: k-row c KC + i (256 / C) + lane / (C / 4), columns 4 (lane % (C / 4)).
    auto off_k = [&](uint32_t row0, uint32_t ld, int i, int c) {
        return (((row0 + (uint32_t)i) * ld + (uint32_t)(c * RKC)) + 4u * (uint32_t)lane) * 4u;
    };
    auto off_o = [&](uint32_t col0, uint32_t ld, int C, int i, int c) {
        const uint32_t kr = (uint32_t)(c * RKC + i * (256 / C) + lane / (C / 4));
        return (kr * ld + col0 + 4u * (uint32_t)(lane % (C / 4))) * 4u;
    };
    auto issue = [&](int c) {
        const int s = c % NS;
        const bool live = c < nck;
#pragma unroll
        for (int q = 0; q < OPS; ++q) {
            const int u = wave + 4 * q;  // wave-uniform
            if (u < TR) {
                const uint32_t dst = ring0 + (uint32_t)(s * ST) * 4u + (RS::AK ? (uint32_t)(u * AS) * 4u : (uint32_t)u * 1024u);
                const uint32_t off = RS::AK ? off_k((uint32_t)r0, K, u, c) : off_o((uint32_t)r0, M, TR, u, c);
                dma16(rsa, dst, live ? off : kOOBf);
            } else {
                const int i = u - TR;
                const uint32_t dst = ring0 + (uint32_t)(s * ST + SA) * 4u + (RS::BK ? (uint32_t)(i * AS) * 4u : (uint32_t)i * 1024u);
                const uint32_t off = RS::BK ? off_k((uint32_t)c0, K, i, c) : off_o((uint32_t)c0, N, TC, i, c);
                dma16(rsb, dst, live ? off : kOOBf);
            }
        }
    };

    const bool idle = r0 + 64 * wave / TC >= m;  // every row of this wave lies past m
    float acc = 0.0f;
#pragma unroll
    for (int c = 0; c < NS - 1; ++c) issue(c);
    for (int c = 0; c < nck; ++c) {
        wait_vmcnt<(NS - 2) * OPS>();  // this wave's units of chunk c have landed
        __syncthreads();               // ... and every wave's; chunk c - 1 is no longer read
        issue(c + NS - 1);             // into chunk c - 1's stage
        if (idle) continue;
        const float *sa = ring + (c % NS) * ST, *sb = sa + SA;
        auto a_at = [&](int kk) -> const float * { return RS::AK ? sa + tr * AS + kk : sa + kk * TR + tr; };
        auto b_at = [&](int kk) -> const float * { return RS::BK ? sb + tc * AS + kk : sb + kk * TC + tc; };
        const int64_t k0 = (int64_t)c * RKC;
        if (k0 + RKC <= k) {
            float xa0[G], xb0[G], xa1[G], xb1[G];
            auto rd = [&](float *xa, float *xb, int kk) {
#pragma unroll
                for (int i = 0; i < G; i += 4) {
                    if constexpr (RS::AK) {
                        const float4 v = *reinterpret_cast<const float4 *>(a_at(kk + i));
                        xa[i] = v.x;
                        xa[i + 1] = v.y;
                        xa[i + 2] = v.z;
                        xa[i + 3] = v.w;
                    } else {
#pragma unroll
                        for (int j = 0; j < 4; ++j) xa[i + j] = *a_at(kk + i + j);
                    }
                    if constexpr (RS::BK) {
                        const float4 u = *reinterpret_cast<const float4 *>(b_at(kk + i));
                        xb[i] = u.x;
                        xb[i + 1] = u.y;
                        xb[i + 2] = u.z;
                        xb[i + 3] = u.w;
                    } else {
#pragma unroll
                        for (int j = 0; j < 4; ++j) xb[i + j] = *b_at(kk + i + j);
                    }
                }
            };
            auto fm = [&](const float *xa, const float *xb) {
#pragma unroll
                for (int i = 0; i < G; ++i) acc = __builtin_fmaf(xa[i], xb[i], acc);
            };
            rd(xa0, xb0, 0);
            for (int kk = 0; kk < RKC; kk += 2 * G) {
                rd(xa1, xb1, kk + G);
                __builtin_amdgcn_sched_barrier(0);
                fm(xa0, xb0);
                rd(xa0, xb0, kk + 2 * G);  // at the chunk's end: read, not used
                __builtin_amdgcn_sched_barrier(0);
                fm(xa1, xb1);
            }
        } else {
            const int kc = (int)(k - k0);
            for (int kk = 0; kk < kc; ++kk) acc = __builtin_fmaf(*a_at(kk), *b_at(kk), acc);
        }
    }
    wait_vmcnt<0>();  // no DMA in flight past this point
    const int64_t r = r0 + tr, c = c0 + tc;
    if (r < m && c < n) out[r * n + c] = acc;
}

// Every byte offset the chain kernels form (including the past-the-row ones
// above, up to a chunk and a tile beyond each operand) stays below 2^31.
bool chain_fits(int64_t m, int64_t k, int64_t n) {
    const int64_t lim = (int64_t)1 << 29;  // floats
    return (m + 64) * (k + 1024) < lim && (k + 1024) * (n + 128) < lim;
}

// The ring kernel's 16-byte DMA pieces: aligned operands, and every row
// along which pieces are taken a multiple of 4 floats long.  At n <= 16 with
// B stored along the outputs (one LDS read per k-step and element) the four
// waves' reads outweigh the latency the ring hides, and the register-staged
// kernel stays (MI355X, us, ring / register-staged: 512x4096x16 34.3 / 27.7;
// 8x1024x1024 9.7 / 13.2, 1x4096x4096 26.0 / 45.6, 16x4096x4096 35.5 / 49;
// C = A.B^T 512x4096x16 25.8 / 27.0).
bool ring_ok(int v, const float *a, const float *b, int64_t m, int64_t k, int64_t n) {
    if (!aligned(a, 16) || !aligned(b, 16)) return false;
    if (v != MM_ABT && n <= 16) return false;
    if (v == MM_ATB) return m % 4 == 0 && n % 4 == 0;
    if (v == MM_ABT) return k % 4 == 0;
    return k % 4 == 0 && n % 4 == 0;
}

template <int V>
int launch_ring(const float *a, const float *b, float *out, int64_t m, int64_t k, int64_t n, hipStream_t s) {
    const int tc = n > 16 ? 32 : (n > 8 ? 16 : 8);
    const int64_t gx = cdiv(n, tc), gy = cdiv(m, TH / tc);
    if (gx > 0x7fffffff || gy > 65535)
        return fail(RQ_ERR_SHAPE, "matmul grid too large (m=%lld n=%lld)", (long long)m, (long long)n);
    const dim3 grid((unsigned)gx, (unsigned)gy);
    switch (tc) {
    case 32: hipLaunchKernelGGL((k_matmul_f32_ring<V, 32>), grid, dim3(TH), 0, s, a, b, out, m, k, n); break;
    case 16: hipLaunchKernelGGL((k_matmul_f32_ring<V, 16>), grid, dim3(TH), 0, s, a, b, out, m, k, n); break;
    default: hipLaunchKernelGGL((k_matmul_f32_ring<V, 8>), grid, dim3(TH), 0, s, a, b, out, m, k, n); break;
    }
    RQ_LAUNCH_CHECK();
    return RQ_OK;
}

template <int V, bool AH = false>
int launch_chain(const void *a, const float *b, float *out, int64_t m, int64_t k, int64_t n, hipStream_t s) {
    const int tc = n >= 64 ? 64 : (n > 16 ? 32 : (n > 8 ? 16 : 8));
    const int64_t gx = cdiv(n, tc), gy = cdiv(m, TH / tc);
    if (gx > 0x7fffffff || gy > 65535)
        return fail(RQ_ERR_SHAPE, "matmul grid too large (m=%lld n=%lld)", (long long)m, (long long)n);
    const dim3 grid((unsigned)gx, (unsigned)gy);
    switch (tc) {
    case 64: hipLaunchKernelGGL((k_matmul_f32_chain<V, 64, AH>), grid, dim3(TH), 0, s, a, b, out, m, k, n); break;
    case 32: hipLaunchKernelGGL((k_matmul_f32_chain<V, 32, AH>), grid, dim3(TH), 0, s, a, b, out, m, k, n); break;
    case 16: hipLaunchKernelGGL((k_matmul_f32_chain<V, 16, AH>), grid, dim3(TH), 0, s, a, b, out, m, k, n); break;
    default: hipLaunchKernelGGL((k_matmul_f32_chain<V, 8, AH>), grid, dim3(TH), 0, s, a, b, out, m, k, n); break;
    }
    RQ_LAUNCH_CHECK();
    return RQ_OK;
}

}  // namespace

int launch_matmul_f32(int variant, const float *a, const float *b, float *out, int64_t m, int64_t k, int64_t n,
                      hipStream_t s) {
    if (m == 0 || n == 0) return RQ_OK;
    const int64_t gx = cdiv(n, BN), gy = cdiv(m, BM);
    // The chain kernels for few outputs or few tiles with more than a few
    // k-steps, measured (MI355X, us, chain / tiled, C = A.B): 8x1024x1024
    // 9.7 / 86, 1x4096x16 22.5 / 335, 16x4096x4096 35.5 / 342, 64x1024x1024
    // 9.9 / 86; with more outputs the tiled kernel's reuse wins (256x1024x4096
    // 356 / 74, 512^3 48 / 38), and at k = 16 its one step (1x16x4096 6.2 / 3.3).
    if (k > 64 && (m * n <= 65536 || gx * gy < 64) && chain_fits(m, k, n)) {
        if (ring_ok(variant, a, b, m, k, n)) {
            switch (variant) {
            case MM_AB: return launch_ring<MM_AB>(a, b, out, m, k, n, s);
            case MM_ABT: return launch_ring<MM_ABT>(a, b, out, m, k, n, s);
            case MM_ATB: return launch_ring<MM_ATB>(a, b, out, m, k, n, s);
            default: break;
            }
        }
        switch (variant) {
        case MM_AB: return launch_chain<MM_AB>(a, b, out, m, k, n, s);
        case MM_ABT: return launch_chain<MM_ABT>(a, b, out, m, k, n, s);
        case MM_ATB: return launch_chain<MM_ATB>(a, b, out, m, k, n, s);
        default: return fail(RQ_ERR_INVALID_ARGUMENT, "unknown matmul variant %d", variant);
        }
    }
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

// C = A.B with A fp16 (exactly widened), where the register-staged chain
// kernel serves the shape (few outputs, n <= 16, k > 64); RQ_ERR_UNSUPPORTED
// (nothing launched) otherwise, and the caller widens A itself.
int launch_matmul_f32_ah(const _Float16 *a, const float *b, float *out, int64_t m, int64_t k, int64_t n,
                         hipStream_t s) {
    if (m == 0 || n == 0) return RQ_OK;
    const int64_t gx = cdiv(n, BN), gy = cdiv(m, BM);
    if (!(k > 64 && (m * n <= 65536 || gx * gy < 64) && chain_fits(m, k, n)) || n > 16) return RQ_ERR_UNSUPPORTED;
    return launch_chain<MM_AB, true>(a, b, out, m, k, n, s);
}

}  // namespace rq
