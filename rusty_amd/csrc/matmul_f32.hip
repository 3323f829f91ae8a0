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
template <int V, int TC>
__global__ __launch_bounds__(TH) void k_matmul_f32_chain(const float *__restrict__ a, const float *__restrict__ b,
                                                         float *__restrict__ out, int64_t m, int64_t k, int64_t n) {
    constexpr int TR = TH / TC;
    constexpr int KC = TC == 16 || TC == 32 ? 512 : 256;  // 64-80 KiB of LDS per chunk
    constexpr int AS = KC + 4;                       // padded A row (floats)
    constexpr int NA = TR * KC / TH, NB = KC * TC / TH;  // chunk elements per thread
    constexpr int G = 32;                            // k-steps per register set of the chains
    // (+ G: the chains' reads one register set past the chunk stay inside the arrays)
    __shared__ __attribute__((aligned(16))) float As[TR * AS + G];
    __shared__ __attribute__((aligned(16))) float Bs[TC * AS + G];
    const int t = threadIdx.x;
    const int64_t r0 = (int64_t)blockIdx.y * TR, c0 = (int64_t)blockIdx.x * TC;
    const int tr = t / TC, tc = t % TC;  // this thread's output
    // chunk element e of this thread: A (row, k) and B (k, column) within the chunk
    auto a_at = [&](int e, int &r, int &kk) {
        const int i = t + TH * e;
        if constexpr (V == MM_ATB) { kk = i / TR; r = i % TR; }  // A stored [k, m]: contiguous along rows
        else { r = i / KC; kk = i % KC; }
    };
    auto b_at = [&](int e, int &kk, int &c) {
        const int i = t + TH * e;
        if constexpr (V == MM_ABT) { c = i / KC; kk = i % KC; }  // B stored [n, k]: contiguous along k
        else { kk = i / TC; c = i % TC; }
    };
    float ra[NA], rb[NB];
    auto load = [&](int64_t k0) {
#pragma unroll
        for (int e = 0; e < NA; ++e) {
            int r, kk;
            a_at(e, r, kk);
            ra[e] = raw_a<V>(a, r0 + r, k0 + kk, m, k);
        }
#pragma unroll
        for (int e = 0; e < NB; ++e) {
            int kk, c;
            b_at(e, kk, c);
            rb[e] = raw_b<V>(b, k0 + kk, c0 + c, k, n);
        }
    };
    auto stage = [&](int64_t k0) {
#pragma unroll
        for (int e = 0; e < NA; ++e) {
            int r, kk;
            a_at(e, r, kk);
            As[r * AS + kk] = in_a<V>(r0 + r, k0 + kk, m, k) ? ra[e] : 0.0f;
        }
#pragma unroll
        for (int e = 0; e < NB; ++e) {
            int kk, c;
            b_at(e, kk, c);
            Bs[c * AS + kk] = in_b<V>(k0 + kk, c0 + c, k, n) ? rb[e] : 0.0f;
        }
    };
    float acc = 0.0f;
    if (k > 0) load(0);
    for (int64_t k0 = 0; k0 < k; k0 += KC) {
        stage(k0);
        __syncthreads();
        if (k0 + KC < k) load(k0 + KC);  // in flight while this chunk's chains run
        const float *ar = As + tr * AS, *bc = Bs + tc * AS;
        if (k0 + KC <= k) {
            // two named register sets of G k-steps: the next set's LDS reads are
            // issued (unconditionally) before the current set's fmas
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
                fm(xa0, xb0);
                rd(xa0, xb0, kk + 2 * G);  // at the chunk's end: read, not used
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

template <int V>
int launch_chain(const float *a, const float *b, float *out, int64_t m, int64_t k, int64_t n, hipStream_t s) {
    const int tc = n >= 64 ? 64 : (n > 16 ? 32 : (n > 8 ? 16 : 8));
    const int64_t gx = cdiv(n, tc), gy = cdiv(m, TH / tc);
    if (gx > 0x7fffffff || gy > 65535)
        return fail(RQ_ERR_SHAPE, "matmul grid too large (m=%lld n=%lld)", (long long)m, (long long)n);
    const dim3 grid((unsigned)gx, (unsigned)gy);
    switch (tc) {
    case 64: hipLaunchKernelGGL((k_matmul_f32_chain<V, 64>), grid, dim3(TH), 0, s, a, b, out, m, k, n); break;
    case 32: hipLaunchKernelGGL((k_matmul_f32_chain<V, 32>), grid, dim3(TH), 0, s, a, b, out, m, k, n); break;
    case 16: hipLaunchKernelGGL((k_matmul_f32_chain<V, 16>), grid, dim3(TH), 0, s, a, b, out, m, k, n); break;
    default: hipLaunchKernelGGL((k_matmul_f32_chain<V, 8>), grid, dim3(TH), 0, s, a, b, out, m, k, n); break;
    }
    RQ_LAUNCH_CHECK();
    return RQ_OK;
}

}  // namespace

int launch_matmul_f32(int variant, const float *a, const float *b, float *out, int64_t m, int64_t k, int64_t n,
                      hipStream_t s) {
    if (m == 0 || n == 0) return RQ_OK;
    const int64_t gx = cdiv(n, BN), gy = cdiv(m, BM);
    // The chain kernel for few outputs or few tiles with more than a few
    // k-steps, measured (MI355X, us, chain / tiled, C = A.B): 8x1024x1024
    // 23.5 / 86, 1x4096x16 45 / 335, 16x4096x4096 88 / 342, 64x1024x1024
    // 24 / 86; with more outputs the tiled kernel's reuse wins (256x1024x4096
    // 356 / 88, 512^3 48 / 45), and at k = 16 its one step (1x16x4096 6.2 / 3.3).
    if (k > 64 && (m * n <= 65536 || gx * gy < 64)) {
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

}  // namespace rq
