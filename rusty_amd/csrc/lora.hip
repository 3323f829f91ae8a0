// Linear::forward with a LoRA adapter (rusty-graph/src/lib.rs:69-83):
//   out = x . W + (x . A) . B,   A [in, rank], B [rank, out] (LoRAAdapter,
//   lib.rs:17-22), added unscaled as the reference does (its alpha is unused).
// Here W is the quantized [out, in] weight, so the first term is rq_qmatmul's
// fused dequant product.  The adapter's two products keep the reference's
// arithmetic: f32 operands, one fma accumulator per output over k ascending
// (the f32 matmul kernel, matmul_f32.hip, for x . A; the same chain over
// the rank for (x . A) . B), then one f32 add per output -- so with W's term
// exactly zero the result equals the reference's f32 path bit for bit.
// Launches: [x widened to f32, where the chain kernel does not take fp16 x
// itself], t = x . A, the fused product into f32, then
// y = main + t . B (rounded to y's dtype) in one pass.  The adapter's work is
// (m . in + m . out) . rank fmas and m . (rank + out) + rank . out floats of
// traffic: small next to the weight for the ranks adapters use (<= 64).
//
// The k-ascending chain of x . A is latency-bound: in_features dependent fmas
// per output (~16 us at in = 4096, whatever m), 3-6x the fused product it
// is added to at decode sizes.  RQ_LORA_TREE (rank <= 64) computes x . A as
// a reduction tree instead: slices of 256 k per block, a short fma chain per
// thread, a fixed-order sum over the block's threads, the slices added in
// order by the output pass -- deterministic, within f32 rounding of the exact
// product, but not the reference's bit pattern.  The fused product itself is
// the same in both modes.
#include <algorithm>
#include <type_traits>

#include "common.hpp"

namespace rq {
namespace {

constexpr int TH = 256;

__global__ __launch_bounds__(TH) void k_widen_f16(const _Float16 *__restrict__ x, float *__restrict__ out, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * TH + threadIdx.x; i < n; i += (int64_t)gridDim.x * TH)
        out[i] = (float)x[i];
}

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// RQ_LORA_TREE's x . A: block (g, s) takes rows g RM .. g RM + RM - 1 of x
// and k slice s (TH J values of k); thread tt multiplies k = s TH J + j TH + tt
// for j < J, its RM RK products accumulated over j in one fma chain each
// (every j's loads issued before the first fma); the block's TH partials of
// every (row, r) are then summed in a fixed order (through LDS: P = TH /
// (RM RK) lanes per value each add every P-th partial, then DPP steps over
// those P lanes) and the slice's sum goes to part[(row KS + s) rank + r].
// VA (rank % 4 == 0, A 16-byte aligned): a k's rank values as 16-byte loads.
// Rows past m recompute row m - 1 and write nothing; r past rank multiplies
// zeros.
template <int RM, int RK, bool F16, int J, bool VA>
__global__ __launch_bounds__(TH) void k_lora_xa(const void *__restrict__ xv, const float *__restrict__ a,
                                                float *__restrict__ part, int64_t m, int64_t K, int rank, int KS) {
    constexpr int V = RM * RK, P = TH / V;
    static_assert(TH % V == 0 && (P == 4 || P == 16), "4 or 16 lanes per value");
    __shared__ float red[V][TH + 1];
    const int tt = threadIdx.x, s = blockIdx.y;
    const int64_t i0 = (int64_t)blockIdx.x * RM, k0 = (int64_t)s * TH * J;
    float av[J][RK], xk[J][RM];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int64_t k = k0 + (int64_t)j * TH + tt;
        const bool live = k < K;
        if constexpr (VA) {
            const float4 *ar = reinterpret_cast<const float4 *>(a + (live ? k : 0) * rank);
#pragma unroll
            for (int r4 = 0; r4 < RK / 4; ++r4) {
                const float4 v = 4 * r4 < rank ? ar[r4] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                av[j][4 * r4] = v.x;
                av[j][4 * r4 + 1] = v.y;
                av[j][4 * r4 + 2] = v.z;
                av[j][4 * r4 + 3] = v.w;
            }
        } else {
#pragma unroll
            for (int r = 0; r < RK; ++r) av[j][r] = r < rank ? a[(live ? k : 0) * rank + r] : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < RM; ++i) {
            const int64_t row = i0 + i < m ? i0 + i : m - 1, o = row * K + (live ? k : 0);
            const float x = F16 ? (float)static_cast<const _Float16 *>(xv)[o] : static_cast<const float *>(xv)[o];
            xk[j][i] = live ? x : 0.0f;
        }
    }
    float acc[V];
#pragma unroll
    for (int v = 0; v < V; ++v) acc[v] = 0.0f;
#pragma unroll
    for (int j = 0; j < J; ++j)
#pragma unroll
        for (int i = 0; i < RM; ++i)
#pragma unroll
            for (int r = 0; r < RK; ++r) acc[i * RK + r] = __builtin_fmaf(xk[j][i], av[j][r], acc[i * RK + r]);
#pragma unroll
    for (int v = 0; v < V; ++v) red[v][tt] = acc[v];
    __syncthreads();
    const int v = tt / P, q = tt % P;
    float sum = 0.0f;
#pragma unroll 8
    for (int e = 0; e < V; ++e) sum += red[v][e * P + q];
    // the P lanes of value v are one aligned group of a DPP row
    sum += dpp<0xB1>(sum);  // quad_perm [1,0,3,2]
    sum += dpp<0x4E>(sum);  // quad_perm [2,3,0,1]
    if constexpr (P == 16) {
        sum += dpp<0x141>(sum);  // row_half_mirror
        sum += dpp<0x140>(sum);  // row_mirror
    }
    const int i = v / RK, r = v % RK;
    if (q == 0 && r < rank && i0 + i < m) part[((i0 + i) * KS + s) * rank + r] = sum;
}

// y[i][c] = main[i][c] + sum_r t[i][r] B[r][c], the sum one fma chain from
// zero over r ascending (the f32 matmul's arithmetic for t . B); main may
// alias y when y is f32.  Thread c of block (x, y) takes column x TH + c of
// rows y, y + gridDim.y, ...: with RB > 0 (rank <= RB) it holds its column of
// B in registers across those rows (read once, not once per row: at
// m = 512 x 4096 x rank 16 the per-row reads were 128 MB of cache traffic),
// t's row is a broadcast read.
template <bool F16, int RB>
__global__ __launch_bounds__(TH) void k_lora_out(const float *main, const float *__restrict__ t,
                                                 const float *__restrict__ b, int rank, void *y, int64_t m,
                                                 int64_t n) {
    const int64_t c = (int64_t)blockIdx.x * TH + threadIdx.x;
    if (c >= n) return;
    float bc[RB > 0 ? RB : 1];
    if constexpr (RB > 0) {
#pragma unroll
        for (int r = 0; r < RB; ++r) bc[r] = b[(int64_t)(r < rank ? r : 0) * n + c];
    }
    for (int64_t i = blockIdx.y; i < m; i += gridDim.y) {
        const float *tr = t + i * rank;
        float acc = 0.0f;
        if constexpr (RB > 0) {
            float tv[RB];  // all requested first (clamped index), then the chain
#pragma unroll
            for (int r = 0; r < RB; ++r) tv[r] = tr[r < rank ? r : 0];
#pragma unroll
            for (int r = 0; r < RB; ++r) {
                const float f = __builtin_fmaf(tv[r], bc[r], acc);
                acc = r < rank ? f : acc;
            }
        } else {
            for (int r = 0; r < rank; ++r) acc = __builtin_fmaf(tr[r], b[(int64_t)r * n + c], acc);
        }
        const int64_t o = i * n + c;
        const float v = main[o] + acc;
        if constexpr (F16) static_cast<_Float16 *>(y)[o] = (_Float16)v;
        else static_cast<float *>(y)[o] = v;
    }
}

// The tree's output pass: as k_lora_out (rank <= RB), with t[i][r] the sum
// over s < KS of part[(i KS + s) rank + r], s ascending.  Block (x, y) takes
// rows [y rpb, (y + 1) rpb) in chunks of up to RC rows: the chunk's KS rank
// partials per row are contiguous, staged in LDS with one coalesced load
// (the chunk's main values requested with them), summed per (row, r) by the
// block's threads into LDS, then every thread finishes its column of each
// row -- two barriers per chunk, not per row.
constexpr int kTreeParts = 8192;  // partials the output pass stages per chunk
constexpr int kTreeRows = 8;      // rows per chunk (RC)
template <bool F16, int RB>
__global__ __launch_bounds__(TH) void k_lora_out_tree(const float *main, const float *__restrict__ part, int KS,
                                                      const float *__restrict__ b, int rank, void *y, int64_t m,
                                                      int64_t n, int64_t rpb, int rc_max) {
    constexpr int RC = kTreeRows;
    __shared__ float pbuf[kTreeParts];
    __shared__ float tsh[RC][RB];
    const int tt = threadIdx.x;
    const int64_t c = (int64_t)blockIdx.x * TH + tt;
    const bool live = c < n;
    const int np = KS * rank;
    float bc[RB];
#pragma unroll
    for (int r = 0; r < RB; ++r) bc[r] = live ? b[(int64_t)(r < rank ? r : 0) * n + c] : 0.0f;
    const int64_t r_begin = (int64_t)blockIdx.y * rpb, r_end = r_begin + rpb < m ? r_begin + rpb : m;
    for (int64_t r0 = r_begin; r0 < r_end; r0 += rc_max) {
        const int rc = (int)(r0 + rc_max < r_end ? rc_max : r_end - r0);
        float mv[RC];
#pragma unroll
        for (int j = 0; j < RC; ++j) mv[j] = live && j < rc ? main[(r0 + j) * n + c] : 0.0f;
        const float *pr = part + r0 * np;
        for (int e = tt; e < rc * np; e += TH) pbuf[e] = pr[e];
        __syncthreads();
        for (int pq = tt; pq < rc * rank; pq += TH) {
            const int j = pq / rank, r = pq % rank;
            float tv = pbuf[j * np + r];
            for (int sl = 1; sl < KS; ++sl) tv += pbuf[j * np + sl * rank + r];
            tsh[j][r] = tv;
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < RC; ++j) {
            if (j >= rc) break;
            float acc = 0.0f;
#pragma unroll
            for (int r = 0; r < RB; ++r) {
                const float f = __builtin_fmaf(tsh[j][r < rank ? r : 0], bc[r], acc);
                acc = r < rank ? f : acc;
            }
            if (live) {
                const int64_t o = (r0 + j) * n + c;
                const float v = mv[j] + acc;
                if constexpr (F16) static_cast<_Float16 *>(y)[o] = (_Float16)v;
                else static_cast<float *>(y)[o] = v;
            }
        }
        __syncthreads();  // pbuf and tsh are rewritten for the next chunk
    }
}

unsigned grid_for(int64_t n) { return (unsigned)std::max<int64_t>(1, std::min<int64_t>(cdiv(n, TH), 16384)); }

// RQ_LORA_TREE serves adapters up to this rank (wider ones take the chain)
constexpr int64_t kTreeRank = 64;
// k values per slice of the tree's x . A at J = 1
constexpr int64_t kSlice = TH;

bool tree_mode(unsigned flags, int64_t rank, int64_t k_in) {
    return (flags & RQ_LORA_TREE) && rank > 0 && rank <= kTreeRank && k_in > 0 &&
           cdiv(k_in, kSlice) * rank <= kTreeParts;
}

size_t lora_workspace(int64_t m, int64_t k_in, int64_t n_out, int64_t rank, rq_dtype x_dtype, rq_dtype y_dtype,
                      unsigned flags) {
    if (m < 0 || k_in < 0 || n_out < 0 || rank < 0) return 0;
    // chain: [x f32][t]; tree: the partials of at most cdiv(k_in, 256) slices
    const int64_t adapter = tree_mode(flags, rank, k_in) ? m * rank * std::max<int64_t>(1, cdiv(k_in, kSlice))
                                                   : (x_dtype == RQ_F16 ? m * k_in : 0) + m * rank;
    const int64_t floats = adapter + (y_dtype == RQ_F16 ? m * n_out : 0);
    return (size_t)floats * 4 + 3 * 256;  // + alignment of each part to 256 bytes
}

// t = x . A as the tree's slice partials part[m][KS][rank]; returns KS.
int launch_lora_xa(const void *x, rq_dtype xt, const float *a, float *part, int64_t m, int64_t K, int64_t rank,
                   int num_cus, hipStream_t s, int *ks_out) {
    const bool rows4 = rank <= 16 && m > 1;  // 4 rows x 16 ranks per block, else 1 row x 16 or 64
    const int64_t G = cdiv(m, rows4 ? 4 : 1), S1 = std::max<int64_t>(1, cdiv(K, kSlice));
    // the most k per thread (all loaded before the fmas; capped so the
    // registers hold them) that still gives ~2 blocks per CU
    const int jmax = rank > 16 ? 2 : (rows4 ? 4 : 8);
    int J = 1;
    while (J < jmax && G * cdiv(S1, 2 * J) >= 2 * num_cus) J *= 2;
    const int64_t KS = std::max<int64_t>(1, cdiv(K, kSlice * J));
    if (G > 0x7fffffff || KS > 65535) return fail(RQ_ERR_SHAPE, "adapter product too large for the tree");
    const dim3 grid((unsigned)G, (unsigned)KS);
    const bool f16 = xt == RQ_F16, va = rank % 4 == 0 && aligned(a, 16);
    auto go = [&](auto rm, auto rk, auto jj, auto vv) {
        constexpr int RM = decltype(rm)::value, RK = decltype(rk)::value, JJ = decltype(jj)::value;
        constexpr bool VA = decltype(vv)::value;
        if (f16) hipLaunchKernelGGL((k_lora_xa<RM, RK, true, JJ, VA>), grid, dim3(TH), 0, s, x, a, part, m, K, (int)rank, (int)KS);
        else hipLaunchKernelGGL((k_lora_xa<RM, RK, false, JJ, VA>), grid, dim3(TH), 0, s, x, a, part, m, K, (int)rank, (int)KS);
    };
    auto by_va = [&](auto rm, auto rk, auto jj) {
        if (va) go(rm, rk, jj, std::true_type{});
        else go(rm, rk, jj, std::false_type{});
    };
    auto by_j = [&](auto rm, auto rk) {
        if (J == 1) by_va(rm, rk, std::integral_constant<int, 1>{});
        else if (J == 2) by_va(rm, rk, std::integral_constant<int, 2>{});
        else if (J == 4) by_va(rm, rk, std::integral_constant<int, 4>{});
        else by_va(rm, rk, std::integral_constant<int, 8>{});
    };
    if (rows4) by_j(std::integral_constant<int, 4>{}, std::integral_constant<int, 16>{});
    else if (rank <= 16) by_j(std::integral_constant<int, 1>{}, std::integral_constant<int, 16>{});
    else by_j(std::integral_constant<int, 1>{}, std::integral_constant<int, 64>{});
    RQ_LAUNCH_CHECK();
    *ks_out = (int)KS;
    return RQ_OK;
}

int lora_run(rq_ctx *ctx, const rq_qweight *w, const void *x, rq_dtype x_dtype, const float *lora_a,
             const float *lora_b, int64_t rank, void *y, rq_dtype y_dtype, int64_t m, unsigned flags, void *workspace,
             size_t workspace_bytes, rq_stream stream) {
    RQ_ENTER(ctx);
    int st = check_qweight(w);
    if (st != RQ_OK) return st;
    if ((x_dtype != RQ_F16 && x_dtype != RQ_F32) || (y_dtype != RQ_F16 && y_dtype != RQ_F32))
        return fail(RQ_ERR_INVALID_ARGUMENT, "dtype must be RQ_F16 or RQ_F32");
    if (flags & ~RQ_LORA_TREE) return fail(RQ_ERR_INVALID_ARGUMENT, "unknown flags 0x%x", flags);
    if (m < 0 || rank < 0) return fail(RQ_ERR_SHAPE, "negative m or rank");
    const int64_t K = w->k_in, N = w->n_out;
    int64_t t;
    if (!mul_ok(m, K, &t) || !mul_ok(m, N, &t) || !mul_ok(m, rank, &t) || !mul_ok(rank, N, &t) ||
        !mul_ok(rank, K, &t) || !mul_ok(m * rank, std::max<int64_t>(1, cdiv(K, kSlice)), &t))
        return fail(RQ_ERR_SHAPE, "shape overflows");
    if (rank > 0x7fffffff || cdiv(N, TH) > 0x7fffffff) return fail(RQ_ERR_SHAPE, "adapter rank or n_out too large");
    if (m == 0 || N == 0) return RQ_OK;
    if (!y || (K > 0 && !x)) return fail(RQ_ERR_INVALID_ARGUMENT, "null activation pointer");
    // (an empty reduction, k_in = 0, gives A no elements: it may be null)
    if (rank > 0 && ((K > 0 && !lora_a) || !lora_b)) return fail(RQ_ERR_INVALID_ARGUMENT, "null adapter pointer");
    const size_t need = lora_workspace(m, K, N, rank, x_dtype, y_dtype, flags);
    if ((need > 0 && !workspace) || workspace_bytes < need)
        return fail(RQ_ERR_INVALID_ARGUMENT, "workspace of %zu bytes, %zu needed", workspace_bytes, need);
    hipStream_t s = pick(ctx, stream);
    // carve the workspace: chain [x f32][t][main f32], tree [partials][main f32]
    char *p = static_cast<char *>(workspace);
    auto carve = [&p](int64_t floats) {
        p = reinterpret_cast<char *>((reinterpret_cast<uintptr_t>(p) + 255) & ~uintptr_t(255));
        float *r = reinterpret_cast<float *>(p);
        p += floats * 4;
        return r;
    };
    const bool tree = tree_mode(flags, rank, K);
    int KS = 1;
    float *tv;
    if (tree) {
        tv = carve(m * rank * cdiv(K, kSlice));
        if ((st = launch_lora_xa(x, x_dtype, lora_a, tv, m, K, rank, ctx->num_cus, s, &KS)) != RQ_OK) return st;
    } else {
        float *w32 = x_dtype == RQ_F16 ? carve(m * K) : nullptr;
        tv = carve(m * rank);
        // t = x . A [m, rank]: one fma chain per output, k ascending.  fp16 x:
        // the chain kernel widens it while staging where it serves the shape,
        // else x is widened to f32 first (exact either way).
        st = x_dtype == RQ_F16 ? launch_matmul_f32_ah(static_cast<const _Float16 *>(x), lora_a, tv, m, K, rank, s)
                               : RQ_ERR_UNSUPPORTED;
        if (st == RQ_ERR_UNSUPPORTED) {
            const float *xf = static_cast<const float *>(x);
            if (x_dtype == RQ_F16) {
                if (m * K > 0) {
                    hipLaunchKernelGGL(k_widen_f16, dim3(grid_for(m * K)), dim3(TH), 0, s,
                                       static_cast<const _Float16 *>(x), w32, m * K);
                    RQ_LAUNCH_CHECK();
                }
                xf = w32;
            }
            st = launch_matmul_f32(MM_AB, xf, lora_a, tv, m, K, rank, s);
        }
        if (st != RQ_OK) return st;
    }
    float *mainv = y_dtype == RQ_F16 ? carve(m * N) : static_cast<float *>(y);
    // the fused dequant product, f32
    if ((st = qmatmul_dispatch(ctx, *w, x, x_dtype, mainv, RQ_F32, m, gemm_workspace(ctx, s), s)) != RQ_OK) return st;
    // y = main + t . B [m, n_out]: enough row groups for ~4 blocks per CU,
    // each thread's B column read once per row group
    const int64_t gxl = cdiv(N, TH);
    const int64_t gyl = std::max<int64_t>(1, std::min<int64_t>({m, 65535, cdiv(4 * ctx->num_cus, gxl)}));
    const dim3 grid((unsigned)gxl, (unsigned)gyl);
    auto go = [&](auto f16, auto rb) {
        constexpr bool F = decltype(f16)::value;
        constexpr int R = decltype(rb)::value;
        if constexpr (R > 0) {
            if (tree) {
                const int64_t rpb = cdiv(m, (int64_t)grid.y);
                const int rc = (int)std::min<int64_t>(kTreeRows, kTreeParts / ((int64_t)KS * rank));
                hipLaunchKernelGGL((k_lora_out_tree<F, R>), grid, dim3(TH), 0, s, mainv, tv, KS, lora_b, (int)rank, y,
                                   m, N, rpb, rc);
                return;
            }
        }
        hipLaunchKernelGGL((k_lora_out<F, R>), grid, dim3(TH), 0, s, mainv, tv, lora_b, (int)rank, y, m, N);
    };
    auto go_rb = [&](auto f16) {
        if (rank == 0) go(f16, std::integral_constant<int, 0>{});  // B may be null: nothing is read
        else if (rank <= 16) go(f16, std::integral_constant<int, 16>{});
        else if (rank <= 64) go(f16, std::integral_constant<int, 64>{});
        else go(f16, std::integral_constant<int, 0>{});
    };
    if (y_dtype == RQ_F16) go_rb(std::true_type{});
    else go_rb(std::false_type{});
    RQ_LAUNCH_CHECK();
    return RQ_OK;
}

}  // namespace
}  // namespace rq

using namespace rq;

extern "C" {

size_t rq_qmatmul_lora_workspace(int64_t m, int64_t k_in, int64_t n_out, int64_t rank, rq_dtype x_dtype,
                                 rq_dtype y_dtype) {
    return lora_workspace(m, k_in, n_out, rank, x_dtype, y_dtype, 0);
}

int rq_qmatmul_lora(rq_ctx *ctx, const rq_qweight *w, const void *x, rq_dtype x_dtype, const float *lora_a,
                    const float *lora_b, int64_t rank, void *y, rq_dtype y_dtype, int64_t m, void *workspace,
                    size_t workspace_bytes, rq_stream stream) {
    return lora_run(ctx, w, x, x_dtype, lora_a, lora_b, rank, y, y_dtype, m, 0, workspace, workspace_bytes, stream);
}

size_t rq_qmatmul_lora_ex_workspace(int64_t m, int64_t k_in, int64_t n_out, int64_t rank, rq_dtype x_dtype,
                                    rq_dtype y_dtype, unsigned flags) {
    return lora_workspace(m, k_in, n_out, rank, x_dtype, y_dtype, flags);
}

int rq_qmatmul_lora_ex(rq_ctx *ctx, const rq_qweight *w, const void *x, rq_dtype x_dtype, const float *lora_a,
                       const float *lora_b, int64_t rank, void *y, rq_dtype y_dtype, int64_t m, unsigned flags,
                       void *workspace, size_t workspace_bytes, rq_stream stream) {
    return lora_run(ctx, w, x, x_dtype, lora_a, lora_b, rank, y, y_dtype, m, flags, workspace, workspace_bytes,
                    stream);
}

}  // extern "C"
