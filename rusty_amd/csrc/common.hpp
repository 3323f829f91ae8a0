// Shared helpers of the gfx950 kernels and the C-ABI layer.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>
#include <stddef.h>

#include "rusty_hip.h"

// A device context: the device ordinal, the context's own stream (default
// priority) and the device's compute-unit count.
struct rq_ctx {
    int device;
    hipStream_t stream;
    int num_cus;
    // Split-K workspace of the prefill GEMM (partial sums and per-tile
    // arrival counters), allocated at create; null if that allocation failed.
    float *sk_partials;
    int *sk_counters;
    // Staging area of the prefill GEMM's input preparation (affine scales in
    // [group][row] order, f32 activations cast to fp16), allocated at create.
    void *prep;
};

namespace rq {

// Records a message for rq_last_error() and returns `status`.
int fail(int status, const char *fmt, ...);

// Evaluates a HIP call; on failure records the HIP error and returns RQ_ERR_HIP.
#define RQ_HIP_TRY(expr)                                                              \
    do {                                                                              \
        hipError_t rq_e_ = (expr);                                                    \
        if (rq_e_ != hipSuccess)                                                      \
            return ::rq::fail(RQ_ERR_HIP, "%s: %s (%s:%d)", #expr, hipGetErrorString(rq_e_), \
                              __FILE__, __LINE__);                                    \
    } while (0)

// Launch check: kernel launches report configuration errors via hipGetLastError.
#define RQ_LAUNCH_CHECK() RQ_HIP_TRY(hipGetLastError())

// Clears the calling thread's error message and makes ctx's device current.
int enter(rq_ctx *ctx);
inline hipStream_t pick(rq_ctx *ctx, rq_stream s) { return s ? static_cast<hipStream_t>(s) : ctx->stream; }
// a*b without overflow; false if it does not fit in int64 (or is negative).
bool mul_ok(int64_t a, int64_t b, int64_t *out);
// Validates an rq_qweight descriptor (format, shape, null pointers).
int check_qweight(const rq_qweight *w);

#define RQ_ENTER(ctx)                       \
    do {                                    \
        int rq_st_ = ::rq::enter(ctx);      \
        if (rq_st_ != RQ_OK) return rq_st_; \
    } while (0)

inline bool aligned(const void *p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Launchers implemented in the kernel translation units.  Arguments are
// validated by the C-ABI layer before these are called.
int launch_dequantize(const uint32_t *in, size_t n_words, float *out, size_t n_out, hipStream_t s);
int launch_affine_dequantize(const uint32_t *w, const float *scales, const float *biases, float *out,
                             size_t n, uint32_t group, bool fma, hipStream_t s);
int launch_rowwise_dequantize(const int8_t *q, const float *scales, float *out, int64_t n_rows,
                              int64_t k, hipStream_t s);
int launch_matmul_f32(int variant, const float *a, const float *b, float *out, int64_t m, int64_t k,
                      int64_t n, hipStream_t s);
// C = A.B with fp16 A where the chain kernel takes it directly; RQ_ERR_UNSUPPORTED otherwise.
int launch_matmul_f32_ah(const _Float16 *a, const float *b, float *out, int64_t m, int64_t k, int64_t n,
                         hipStream_t s);
int launch_gemv_decode(const rq_qweight &w, const void *x, rq_dtype xt, void *y, rq_dtype yt, int m, hipStream_t s);
// m = 1..4 decode GEMV that adds its result into an f32 y (y += X . deq(W)^T):
// the residual connection fused into the projection's epilogue.
int launch_gemv_decode_add(const rq_qweight &w, const void *x, float *y, int m, hipStream_t s);
// m = 1 decode GEMV whose activation row is RMSNorm(x) . nw, computed in the
// kernel's prologue from the f32 row x (no separate norm launch); f32 y.
int launch_gemv_decode_norm(const rq_qweight &w, const float *x, const _Float16 *nw, float eps, float *y,
                            hipStream_t s);
int launch_gemv_mfma(const rq_qweight &w, const void *x, rq_dtype xt, void *y, rq_dtype yt, int m, hipStream_t s);
int launch_gemv(const rq_qweight &w, const void *x, rq_dtype xt, void *y, rq_dtype yt, int m,
                int num_cus, hipStream_t s);
// Split-K workspace of the prefill GEMM: kGemmSkFloats f32 partial sums and
// kGemmSkCounters per-tile counters (one 128-byte line each, zero between launches).
constexpr size_t kGemmSkFloats = (size_t)8 << 20;  // 32 MiB
constexpr int kGemmSkCounters = 4096;
// Input-preparation area of the prefill GEMM: affine scales transposed to
// [group][row] (8 bytes per group), then f32 activations cast to fp16 (a
// chunk of rows at a time when they do not fit).
constexpr size_t kGemmPrepBytes = (size_t)64 << 20;  // 64 MiB
struct GemmWorkspace {
    float *partials;  // null: no split-K
    int *counters;
    size_t floats;
    int n_counters;
    void *prep = nullptr;  // null: no affine or f32-activation GEMM (the generic kernel serves them)
    size_t prep_bytes = 0;
};
// The workspace of ctx when work on stream s may use it: the context's own
// stream only (two GEMMs running at once on different streams would share it).
GemmWorkspace gemm_workspace(const rq_ctx *ctx, hipStream_t s);
// The outputs of launch_gemm_qkv_rope (a Llama layer's packed q/k/v projection
// over positions p0 .. of a prompt chunk): this layer's K and V caches
// [n_kv][max_seq][64] fp16 and the rotation table rope[pos * 32 + d] =
// (cos, sin) of position pos and pair d; q goes to the call's q argument.
struct RopeOut {
    const float2 *rope = nullptr;
    _Float16 *kc = nullptr, *vc = nullptr;
    int p0 = 0, n_heads = 0, n_kv = 0, max_seq = 0;
};
int launch_gemm_qkv_rope(const rq_qweight &w, const _Float16 *x, int64_t m, const RopeOut &ro, _Float16 *q,
                         int num_cus, const GemmWorkspace &ws, hipStream_t s);
int launch_gemm(const rq_qweight &w, const void *x, rq_dtype xt, void *y, rq_dtype yt, int64_t m, int num_cus,
                const GemmWorkspace &ws, hipStream_t s);
// Y = (xscale[row] * X[row]) . (scales * W)^T for per-row int8 W and fp16 X
// (xscale: a power of two per activation row); RQ_ERR_UNSUPPORTED outside the
// prefill GEMM's tiles (k_in % 64, alignment).
int launch_gemm_f16_scaled(const rq_qweight &w, const float *scales, const _Float16 *x, const float *xscale,
                           void *y, rq_dtype yt, int64_t m, int num_cus, const GemmWorkspace &ws, hipStream_t s);
// Bytes of the prefill GEMM's scale table of an affine weight (0: none), and
// the launch that builds it (table[g][0][n] = s, table[g][1][n] = b - 1024 s).
size_t affine_prep_bytes(const rq_qweight &w);
int launch_affine_prep(const rq_qweight &w, float *table, hipStream_t s);
// h = fp16(silu(X . deq(gate)^T) * (X . deq(up)^T)) in one GEMM launch, g and
// u rounded to fp16 before the silu*mul (per-row int8, fp16 X, I % 8 == 0, a
// grid that fills the device); RQ_ERR_UNSUPPORTED otherwise.
int launch_gemm_swiglu(const rq_qweight &gate, const rq_qweight &up, const void *x, rq_dtype xt, void *h, int64_t m,
                       int num_cus, const GemmWorkspace &ws, hipStream_t s);
int launch_qlinear_generic(const rq_qweight &w, const void *x, rq_dtype xt, void *y, rq_dtype yt,
                           int64_t m, hipStream_t s);
int launch_swiglu_decode(const rq_qweight &gate, const rq_qweight &up, const void *x, rq_dtype xt, void *h, int m,
                         hipStream_t s);
// SwiGLU gate/up pass over RMSNorm(x) . nw (m = 1, f32 x), h fp16.
int launch_swiglu_decode_norm(const rq_qweight &gate, const rq_qweight &up, const float *x, const _Float16 *nw,
                              float eps, void *h, hipStream_t s);
// The q/k/v projection of one decode step with its rotary epilogue: the
// position (device), the (cos, sin) table rope[p * hd/2 + d], the rotated
// query q (f32 [n_heads][hd]) and this layer's K and V caches
// [n_kv][max_seq][hd] (fp16), which receive the step's rotated key and value
// at the position.
struct RopeDecode {
    const int *pos = nullptr;
    const float2 *rope = nullptr;
    float *q = nullptr;
    _Float16 *kc = nullptr, *vc = nullptr;
    int n_heads = 0, n_kv = 0, hd = 0, max_seq = 0;
};
// m = 1: [q; k; v] = RMSNorm(x) . nw . W^T (W packed q, k, v rows, head_dim
// rows per head), then RoPE (rotate-half pairs d, d + hd/2) on q and k; q
// to rd.q, k and v (fp16) into the caches at *rd.pos.
int launch_gemv_decode_qkv_rope(const rq_qweight &w, const float *x, const _Float16 *nw, float eps,
                                const RopeDecode &rd, hipStream_t s);
// y[n] += sum_k W[n, k] x[k] (m = 1, f32 y) with x the decode attention output
// combined in the prologue from n_split (1, 2, 4 or 8) partial softmaxes per head
// of head_dim elements: partials = o[head][n_split][head_dim] fp16 (each
// split's output, normalised by its own sum l), then (m, l)[head][n_split] float2.
int launch_gemv_decode_attn_add(const rq_qweight &w, const float *partials, int n_split, int head_dim, float *y,
                                hipStream_t s);
int launch_swiglu_mfma(const rq_qweight &gate, const rq_qweight &up, const void *x, rq_dtype xt, void *h, int m,
                       hipStream_t s);
int launch_swiglu_generic(const rq_qweight &gate, const rq_qweight &up, const void *x, rq_dtype xt, void *h,
                          int64_t m, hipStream_t s);
int launch_silu_mul(const void *g, const void *u, void *h, int64_t n, hipStream_t s);
// dX[m, k_in] = dY[m, n_out] . deq(W), W dequantized while staged (f32 fma, ascending n_out).
int launch_qmatmul_dx(const rq_qweight &w, const void *dy, rq_dtype dyt, void *dx, rq_dtype dxt, int64_t m,
                      hipStream_t s);

// Batched prompt kernels of the Llama runner (one launch each over n rows).
// x[s] = f32(embed[tokens[s]]) for s < n.
int launch_embed_rows(const int *tokens, const _Float16 *embed, int H, float *x, int n, hipStream_t s);
// x[s] += y[s] (y may be null), then xn[s] = fp16(rmsnorm(x[s]) * nw) (nw null: add only).
int launch_add_rmsnorm_rows(float *x, const float *y, const _Float16 *nw, float eps, _Float16 *xn, int n, int H,
                            hipStream_t s);
// RoPE of rows p0..p0+n-1 of qkv (f32 [n][(n_heads + 2 n_kv) hd]): q to fp16
// [n][n_heads][hd], k and v (fp16) into one layer's cache [n_kv][max_seq][hd].
int launch_rope_scatter(const float *qkv, const float2 *rope, int p0, int n, int n_heads, int n_kv, int hd,
                        int max_seq, _Float16 *q, _Float16 *kc, _Float16 *vc, hipStream_t s);
// Causal attention of the n queries at positions p0.. (p0 % 32 == 0) over
// cache positions 0..p0+n-1; out fp16 [n][n_heads * hd].
int launch_attn_prefill(const _Float16 *q, const _Float16 *kc, const _Float16 *vc, _Float16 *out, int p0, int n,
                        int n_heads, int n_kv, int hd, int max_seq, hipStream_t s);

// Y = X . deq(W)^T over every kernel family, picked by m, dtypes and shape;
// the prefill GEMM may use ws (split-K partials, input preparation).
int qmatmul_dispatch(rq_ctx *ctx, const rq_qweight &w, const void *x, rq_dtype xt, void *y, rq_dtype yt, int64_t m,
                     const GemmWorkspace &ws, hipStream_t s);

// SwiGLU MLP: argument checks (weights, dtypes, shapes) and the launches over
// a workspace h of 2*m*I fp16 values (see rq_mlp_swiglu).
int swiglu_check(const rq_qweight *gate, const rq_qweight *up, const rq_qweight *down, rq_dtype x_dtype,
                 rq_dtype y_dtype, int64_t m);
int swiglu_run(rq_ctx *ctx, const rq_qweight &gate, const rq_qweight &up, const rq_qweight &down, const void *x,
               rq_dtype x_dtype, void *h, void *y, rq_dtype y_dtype, int64_t m, const GemmWorkspace &ws,
               hipStream_t s);

// Looks up this device's copy of the no-alloc entry point's scratch array
// (once per device; `device` must be current).  A failure is recorded and
// reported by that entry point, not by context creation.
void noalloc_init(int device);

enum MatmulVariant { MM_AB = 0, MM_ABT = 1, MM_ATB = 2 };

}  // namespace rq
