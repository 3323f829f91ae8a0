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

unsigned grid_for(int64_t n) { return (unsigned)std::max<int64_t>(1, std::min<int64_t>(cdiv(n, TH), 16384)); }

}  // namespace
}  // namespace rq

using namespace rq;

extern "C" {

size_t rq_qmatmul_lora_workspace(int64_t m, int64_t k_in, int64_t n_out, int64_t rank, rq_dtype x_dtype,
                                 rq_dtype y_dtype) {
    if (m < 0 || k_in < 0 || n_out < 0 || rank < 0) return 0;
    const int64_t floats = (x_dtype == RQ_F16 ? m * k_in : 0) + m * rank + (y_dtype == RQ_F16 ? m * n_out : 0);
    return (size_t)floats * 4 + 3 * 256;  // + alignment of each part to 256 bytes
}

int rq_qmatmul_lora(rq_ctx *ctx, const rq_qweight *w, const void *x, rq_dtype x_dtype, const float *lora_a,
                    const float *lora_b, int64_t rank, void *y, rq_dtype y_dtype, int64_t m, void *workspace,
                    size_t workspace_bytes, rq_stream stream) {
    RQ_ENTER(ctx);
    int st = check_qweight(w);
    if (st != RQ_OK) return st;
    if ((x_dtype != RQ_F16 && x_dtype != RQ_F32) || (y_dtype != RQ_F16 && y_dtype != RQ_F32))
        return fail(RQ_ERR_INVALID_ARGUMENT, "dtype must be RQ_F16 or RQ_F32");
    if (m < 0 || rank < 0) return fail(RQ_ERR_SHAPE, "negative m or rank");
    const int64_t K = w->k_in, N = w->n_out;
    int64_t t;
    if (!mul_ok(m, K, &t) || !mul_ok(m, N, &t) || !mul_ok(m, rank, &t) || !mul_ok(rank, N, &t) ||
        !mul_ok(rank, K, &t))
        return fail(RQ_ERR_SHAPE, "shape overflows");
    if (rank > 0x7fffffff || cdiv(N, TH) > 0x7fffffff) return fail(RQ_ERR_SHAPE, "adapter rank or n_out too large");
    if (m == 0 || N == 0) return RQ_OK;
    if (!y || (K > 0 && !x)) return fail(RQ_ERR_INVALID_ARGUMENT, "null activation pointer");
    if (rank > 0 && (!lora_a || !lora_b)) return fail(RQ_ERR_INVALID_ARGUMENT, "null adapter pointer");
    const size_t need = rq_qmatmul_lora_workspace(m, K, N, rank, x_dtype, y_dtype);
    if (!workspace || workspace_bytes < need)
        return fail(RQ_ERR_INVALID_ARGUMENT, "workspace of %zu bytes, %zu needed", workspace_bytes, need);
    hipStream_t s = pick(ctx, stream);
    // carve the workspace: [x f32][t][main f32]
    char *p = static_cast<char *>(workspace);
    auto carve = [&p](int64_t floats) {
        p = reinterpret_cast<char *>((reinterpret_cast<uintptr_t>(p) + 255) & ~uintptr_t(255));
        float *r = reinterpret_cast<float *>(p);
        p += floats * 4;
        return r;
    };
    float *w32 = x_dtype == RQ_F16 ? carve(m * K) : nullptr;
    float *tv = carve(m * rank);
    float *mainv = y_dtype == RQ_F16 ? carve(m * N) : static_cast<float *>(y);
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

}  // extern "C"
