/*
 * rusty_hip.h -- C ABI of the MI355X (gfx950) quantized-linear hot path.
 *
 * Drop-in for the op surface of Rusty's `ComputeEngine` on the int8
 * quantized-linear path (rusty-backend/src/lib.rs).  Plain pointers and sizes,
 * no C++ or torch types, bindgen-clean.  All tensor pointers are DEVICE
 * pointers owned by the caller (the reference's caller-allocated `out`
 * convention, rusty-autograd/src/lib.rs:468-477).  Every call returns an
 * rq_status; nothing aborts.  Work is enqueued on a HIP stream (NULL = the
 * context's own stream) and is asynchronous, like the reference's
 * `queue.submit`; completion is observed with rq_sync (the reference's
 * `device.poll(Wait)` inside `UnifiedTensor::to_vec`, lib.rs:215-240).
 * A context is used from one host thread at a time (the reference's Tensor is
 * RefCell-based and single-threaded, rusty-autograd/src/lib.rs:11-17).
 * Degenerate sizes are valid for the dequantizers and the products
 * (rq_qmatmul, rq_mlp_swiglu and its no-alloc variant, rq_qmatmul_lora and
 * _ex, rq_qmatmul_dx): a call with no tokens or no output elements writes
 * nothing; an empty reduction (k_in = 0, or a SwiGLU MLP without intermediate
 * features) writes zeros; a pointer to an operand, adapter or workspace that
 * holds no element may be NULL.  Entry points with stated shape limits (the
 * matrix-core input gradient) keep them.
 */
#ifndef RUSTY_HIP_H
#define RUSTY_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------ */
typedef enum rq_status {
    RQ_OK = 0,
    RQ_ERR_INVALID_ARGUMENT = -1, /* null pointer, bad enum, bad flag        */
    RQ_ERR_SHAPE = -2,            /* sizes inconsistent or out of range      */
    RQ_ERR_UNSUPPORTED = -3,      /* valid request this build does not serve */
    RQ_ERR_HIP = -4,              /* a HIP runtime call failed               */
    RQ_ERR_NO_DEVICE = -5,        /* no gfx950 device with that ordinal      */
    RQ_ERR_ALLOC = -6             /* device or host allocation failed        */
} rq_status;

typedef enum rq_dtype { RQ_F32 = 0, RQ_F16 = 1 } rq_dtype;

/* Quantized weight formats.
 *  RQ_Q_ROWWISE_I8: signed int8 codes q[n,k], one f32 scale per output row:
 *                   W[n,k] = f32(q[n,k]) * scales[n].
 *  RQ_Q_AFFINE_U8 : the reference's MLX-style affine 8-bit format
 *                   (rusty-backend/src/kernels.wgsl:379-400, loaded by
 *                   rusty-loader/src/lib.rs:155-218): unsigned codes u,
 *                   f32 scale and bias per `group` consecutive elements of the
 *                   flattened row-major index i = n*k_in + k:
 *                   W[i] = f32(u[i]) * scales[i/group] + biases[i/group]. */
typedef enum rq_qformat { RQ_Q_ROWWISE_I8 = 0, RQ_Q_AFFINE_U8 = 1 } rq_qformat;

/* A quantized Linear weight in [out, in] ("W[n_out, k_in]", K contiguous)
 * orientation: Y = X . deq(W)^T, the semantics of the reference's `matmul_bt`
 * (kernels.wgsl:234-242).  The reference has no int8 tensor type (its DType
 * is {FP32, FP16}, lib.rs:57-76); quantized weights travel as raw buffer
 * triplets (lib.rs:4939-4946).  This struct is that triplet plus its shape. */
typedef struct rq_qweight {
    const void *codes;    /* device, n_out*k_in bytes, row-major           */
    const float *scales;  /* device, ROWWISE: [n_out]; AFFINE: [n_groups]  */
    const float *biases;  /* device, AFFINE: [n_groups] or NULL (= 0)      */
    int64_t n_out;
    int64_t k_in;
    int32_t format;       /* rq_qformat                                    */
    int32_t group;        /* AFFINE: elements per group (64 in reference)  */
    const float *prep;    /* AFFINE, optional: the table rq_qweight_prepare
                           * built from these scales and biases, or NULL   */
} rq_qweight;

typedef struct rq_ctx rq_ctx;
typedef void *rq_stream; /* a hipStream_t; NULL selects the context stream */

/* ---- context ------------------------------------------------------------
 * Replaces WgpuContext::new (rusty-backend/src/lib.rs:20-47) +
 * ComputeEngine::new (lib.rs:343-4017): selects the device, creates the
 * context's stream (default priority) and a 32.5 MB workspace the prefill
 * GEMM uses for split-K partial sums (if that allocation fails the GEMM just
 * never splits).  Fails with RQ_ERR_NO_DEVICE unless the device is a gfx950. */
int rq_ctx_create(int device, rq_ctx **out);
int rq_ctx_destroy(rq_ctx *ctx);
int rq_ctx_stream(rq_ctx *ctx, rq_stream *out);
/* Number of compute units of the context's device. */
int rq_ctx_num_cus(rq_ctx *ctx, int *out);
/* Blocks until all work on `stream` is done (device.poll(Wait), lib.rs:232). */
int rq_sync(rq_ctx *ctx, rq_stream stream);
/* A bounded device-side delay: one wave waits on the device's constant-rate
 * wall clock for `microseconds` (at most 100000, else RQ_ERR_INVALID_ARGUMENT)
 * and exits.  No counterpart in the reference: a benchmarking aid for drivers
 * that issue launches one at a time (e.g. under a tracer that does not follow
 * graph launches) -- work enqueued behind the delay queues up on the device and
 * then runs back to back, as it does when replayed from a graph. */
int rq_device_delay(rq_ctx *ctx, uint32_t microseconds, rq_stream stream);
/* A measurement aid with no counterpart in the reference: a one-wave kernel
 * stores the device's constant-rate wall clock (a 64-bit tick count) to the
 * device address dst when `stream` reaches it; *ticks_per_second (if not NULL)
 * receives the clock's rate on return.  Unlike HIP events it may be captured
 * in a HIP graph, so a region inside one graph launch can be timed. */
int rq_device_clock(rq_ctx *ctx, uint64_t *dst, uint64_t *ticks_per_second, rq_stream stream);
/* A measurement aid with no counterpart in the reference: the decode GEMV's
 * weight stream without its arithmetic.  Reads `rows` rows of `row_bytes`
 * bytes (a multiple of 16, at most 16384) at `src` (16-byte aligned) with the
 * GEMV's grid (blocks of 256 threads, `rows_per_block` rows each, 1..4; every
 * thread loads 16-byte chunks of each row, non-temporal) and XOR-combines each
 * wave's words.  store != 0: lane 0 of wave r stores the combined value of
 * row r of its block (folded to 2 bytes) to dst[row] -- the GEMV's fp16
 * output; store == 0: dst[row] is written only if that value is all ones
 * (never, in practice), so the loads are consumed and nothing is stored.  dst
 * holds `rows` 2-byte values.  Timed beside the GEMV it gives the one-launch
 * read (and read + store) floor for the same bytes. */
int rq_stream_probe(rq_ctx *ctx, const void *src, size_t row_bytes, size_t rows, int rows_per_block, void *dst,
                    int store, rq_stream stream);
/* A measurement aid with no counterpart in the reference: one wave of 64
 * lanes runs `steps` dependent f32 fmas (acc = fma(acc, a, b)) and stores the
 * 64 results to dst (64 floats).  Timed beside the f32 matmul it gives the
 * one-launch floor of a k-ascending fma chain of the same length (the bound
 * of that kernel where few outputs each walk a long k). */
int rq_fma_chain_probe(rq_ctx *ctx, int64_t steps, float *dst, rq_stream stream);
/* Human-readable name of a status code, and the calling thread's last error
 * message (empty string if none). */
const char *rq_status_string(int status);
const char *rq_last_error(void);

/* ---- memory --------------------------------------------------------------
 * Replaces UnifiedTensor::{new, empty, to_vec} (lib.rs:115-240): device
 * allocation, host->device upload, device->host readback.  Unlike the
 * reference's pooled `empty()` (pool.rs:30-56, stale contents), rq_alloc
 * memory is uninitialised and rq_memset clears it explicitly (with a fill
 * kernel, not a memset node, so it may be captured in a HIP graph). */
int rq_alloc(rq_ctx *ctx, size_t bytes, void **dptr);
int rq_free(rq_ctx *ctx, void *dptr);
int rq_memcpy_h2d(rq_ctx *ctx, void *dst, const void *src, size_t bytes, rq_stream stream);
int rq_memcpy_d2h(rq_ctx *ctx, void *dst, const void *src, size_t bytes, rq_stream stream);
int rq_memcpy_d2d(rq_ctx *ctx, void *dst, const void *src, size_t bytes, rq_stream stream);
int rq_memset(rq_ctx *ctx, void *dst, int value, size_t bytes, rq_stream stream);

/* ---- dequantization --------------------------------------------------- */

/* ComputeEngine::dequantize (lib.rs:4872-4899), kernel kernels.wgsl:153-166:
 * out[4i+j] = f32((input[i] >> 8j) & 0xFF) for i < n_words, 4i+j < n_out
 * (little-endian bytes, unsigned, no scale). */
int rq_dequantize(rq_ctx *ctx, const uint32_t *input, size_t n_words, float *out, size_t n_out,
                  rq_stream stream);

/* ComputeEngine::affine_dequantize (lib.rs:4939-4990), kernel
 * kernels.wgsl:379-400:
 * out[i] = f32(byte_i) * scales[i/group] + biases[i/group], i < n_out.
 * `group` is 64 in the reference (hard-coded at kernels.wgsl:395).
 * Requires n_weight_words >= ceil(n_out/4), n_groups >= ceil(n_out/group).
 * flags: 0 = multiply then add, each rounded to f32 (as the WGSL is written);
 * RQ_AFFINE_FMA = one fused multiply-add (a shader compiler that contracts).
 * Every element of out is written: the reference's 2-D dispatch fallback
 * (lib.rs:4976-4987) leaves elements >= 4,194,240 unwritten; this does not. */
#define RQ_AFFINE_FMA 1u
int rq_affine_dequantize(rq_ctx *ctx, const uint32_t *weight, size_t n_weight_words,
                         const float *scales, const float *biases, size_t n_groups, float *out,
                         size_t n_out, uint32_t group, uint32_t flags, rq_stream stream);

/* Dequantizes any rq_qweight to f32 [n_out, k_in] (ROWWISE: f32(q)*s, one
 * rounding; AFFINE: as rq_affine_dequantize with flags 0).  The load-time
 * step of WeightsContext::upload_quantized (rusty-loader/src/lib.rs:155-218)
 * with the logical [out, in] shape (the reference allocates the packed
 * shape, lib.rs:172-174,206). */
int rq_qweight_dequantize(rq_ctx *ctx, const rq_qweight *w, float *out, rq_stream stream);

/* Load-time preparation of an affine weight for the prefill GEMM: the step
 * WeightsContext::upload_quantized (rusty-loader/src/lib.rs:155-218) runs
 * once per weight at load (there, dequantization to f32).  The GEMM reads an
 * affine weight's scales per k-step and row as a table
 * table[g][0][n] = s[n][g], table[g][1][n] = b[n][g] - 1024 s[n][g]
 * (g < k_in / group, the bias term folded with the fp16 expansion's offset).
 * rq_qweight_prep_bytes gives its size in bytes: 8 * n_out * k_in / group
 * for an affine weight whose group is a multiple of 64 dividing k_in (what
 * the GEMM serves), else 0 (nothing to prepare).  rq_qweight_prepare builds
 * the table into `table` (device, 16-byte aligned, table_bytes >= that size)
 * on `stream` and sets w->prep = table; with a size of 0 it only sets
 * w->prep = NULL.  A weight without a table still works: every GEMM call
 * then builds it again in the context's preparation area (context stream
 * only).  The table depends on the scale and bias values: rebuild it if they
 * change.  No reference counterpart as an entry point. */
size_t rq_qweight_prep_bytes(const rq_qweight *w);
int rq_qweight_prepare(rq_ctx *ctx, rq_qweight *w, void *table, size_t table_bytes, rq_stream stream);

/* ---- f32 matmul family (the reference's per-token GEMMs) ---------------
 * All row-major f32, one f32 sum per output in ascending k, each step a fused
 * multiply-add.  m, k, n as the host derives them from tensor shapes. */

/* ComputeEngine::matmul (lib.rs:4403-4453), kernel `matmul_tiled`
 * kernels.wgsl:7-54: out[m,n] = a[m,k] . b[k,n]. */
int rq_matmul(rq_ctx *ctx, const float *a, const float *b, float *out, int64_t m, int64_t k,
              int64_t n, rq_stream stream);
/* ComputeEngine::matmul_bt (lib.rs:4299-4349), kernels.wgsl:234-242:
 * out[m,n] = a[m,k] . b[n,k]^T. */
int rq_matmul_bt(rq_ctx *ctx, const float *a, const float *b, float *out, int64_t m, int64_t k,
                 int64_t n, rq_stream stream);
/* ComputeEngine::matmul_at (lib.rs:4351-4401), kernels.wgsl:244-252:
 * out[m,n] = a[k,m]^T . b[k,n]. */
int rq_matmul_at(rq_ctx *ctx, const float *a, const float *b, float *out, int64_t m, int64_t k,
                 int64_t n, rq_stream stream);

/* ---- fused quantized linear -------------------------------------------
 * Y[m, n_out] = X[m, k_in] . deq(W)^T, dequantization fused into the
 * product (int8 read straight from HBM, scale applied in registers).  This
 * replaces the reference's two-step path -- load-time affine_dequantize to an
 * f32 weight (rusty-loader/src/lib.rs:209) followed by `matmul` on every
 * forward (Linear::forward, rusty-graph/src/lib.rs:69-70 ->
 * Tensor::matmul, rusty-autograd/src/lib.rs:468-477).
 * x_dtype/y_dtype: RQ_F16 or RQ_F32; accumulation is f32.
 * m <= 16 runs the decode GEMV kernels, larger m the MFMA GEMM.  f32
 * activations keep f32 accuracy up to m = 16: each value is carried as two
 * fp16 terms (the weights as exact code values) after an exact power-of-two
 * scaling -- per 16-value chunk of a row for m <= 2; for 3..16 rows, per
 * 256-k batch whenever a value passes fp16's range (65504) -- so any finite
 * f32 row is served (at 3..16 rows a row whose values all lie below 6.1e-5
 * keeps fp16-subnormal precision); the GEMM rounds them to fp16 (the
 * fp16-MFMA prefill path), each row scaled first by the power of two that
 * puts its largest magnitude in [2^14, 2^15) and its outputs scaled back, so
 * there too any finite row is served, at fp16 accuracy; it rounds affine
 * weights to fp16 likewise.  On the
 * context's own stream (stream NULL) a GEMM with few tokens splits K over
 * more blocks using the context's workspace, so two such calls of one
 * context must not run concurrently (they cannot on one stream); on any
 * other stream it does not split.  A HIP graph captured on the context's
 * stream that holds such GEMMs has the workspace baked in: replay it on the
 * context's stream (or never concurrently with other work of the context). */
int rq_qmatmul(rq_ctx *ctx, const rq_qweight *w, const void *x, rq_dtype x_dtype, void *y,
               rq_dtype y_dtype, int64_t m, rq_stream stream);

/* Linear::forward with a LoRA adapter (rusty-graph/src/lib.rs:69-83; the
 * adapter's tensors LoRAAdapter, lib.rs:17-22):
 *   Y[m, n_out] = X . deq(W)^T + (X . A) . B,
 * A f32 [k_in, rank], B f32 [rank, n_out] (row-major), added unscaled as the
 * reference does.  The adapter's products are f32 with one fma accumulator
 * per output over k ascending, then one f32 add to the fused product (which
 * is computed in f32); Y is rounded to y_dtype once.  rank 0 adds nothing.
 * workspace: device memory of at least rq_qmatmul_lora_workspace(...) bytes
 * (f32 copies of X when it is fp16, X.A, and the fused product when Y is
 * fp16).  Uses the context's GEMM workspace as rq_qmatmul does. */
size_t rq_qmatmul_lora_workspace(int64_t m, int64_t k_in, int64_t n_out, int64_t rank, rq_dtype x_dtype,
                                 rq_dtype y_dtype);
int rq_qmatmul_lora(rq_ctx *ctx, const rq_qweight *w, const void *x, rq_dtype x_dtype, const float *lora_a,
                    const float *lora_b, int64_t rank, void *y, rq_dtype y_dtype, int64_t m, void *workspace,
                    size_t workspace_bytes, rq_stream stream);

/* rq_qmatmul_lora with a choice of adapter arithmetic (no counterpart in the
 * reference, whose only arithmetic is the chain; for callers that want the
 * adapter at decode sizes without its latency).  flags 0: exactly
 * rq_qmatmul_lora.  RQ_LORA_TREE (adapters of rank 1..64): X.A as a
 * reduction tree -- slices of 256 k, a fixed-order sum inside each slice, the
 * slices added in order -- deterministic on a given device (the slice
 * width follows the compute-unit count) and within f32 rounding of the
 * exact product, but not the reference's bit pattern; wider adapters keep
 * the chain.  The k_in-step fma chain per output that reproduces the
 * reference's bits is latency-bound (~16 us at k_in = 4096, whatever m).
 * workspace: at least rq_qmatmul_lora_ex_workspace(..., flags) bytes. */
#define RQ_LORA_TREE 1u
size_t rq_qmatmul_lora_ex_workspace(int64_t m, int64_t k_in, int64_t n_out, int64_t rank, rq_dtype x_dtype,
                                    rq_dtype y_dtype, unsigned flags);
int rq_qmatmul_lora_ex(rq_ctx *ctx, const rq_qweight *w, const void *x, rq_dtype x_dtype, const float *lora_a,
                       const float *lora_b, int64_t rank, void *y, rq_dtype y_dtype, int64_t m, unsigned flags,
                       void *workspace, size_t workspace_bytes, rq_stream stream);

/* MLP::forward (rusty-graph/src/lib.rs:317-323):
 * y = down( silu(x . gate^T) * (x . up^T) ), silu(v) = v / (1 + exp(-v))
 * (kernels.wgsl:104-113; the elementwise product kernels.wgsl:146-151).
 * gate, up: [I, H]; down: [H, I]; x [m, H]; y [m, H].
 * h: caller workspace of 2*m*I fp16 values; on return its first m*I hold the
 * activated intermediate silu(g)*u (rounded to fp16).  For m <= 16 with fp16
 * activations and per-row int8 weights, gate and up are read in one fused
 * pass with the silu*mul epilogue. */
int rq_mlp_swiglu(rq_ctx *ctx, const rq_qweight *gate, const rq_qweight *up, const rq_qweight *down, const void *x,
                  rq_dtype x_dtype, void *h, void *y, rq_dtype y_dtype, int64_t m, rq_stream stream);

/* No counterpart in the reference: rq_mlp_swiglu for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops that
 * forbid hipMalloc).  Same kernels as rq_mlp_swiglu, but the intermediate h
 * lives in a library-owned device array of 8 MiB per device (held until the
 * process ends) instead of a caller workspace, so the call allocates nothing,
 * and none of its GEMMs (gate/up or down) uses the context's workspace: they
 * never split K (so a prefill result may differ from rq_mlp_swiglu's in the
 * summation order where that one splits), and f32 activations or affine
 * weights without a prepared table (rq_qweight_prepare) at m > 16 take the
 * generic kernel.
 * Limit: 4 * m * intermediate <= 8 MiB (m * intermediate <= 2,097,152), else
 * RQ_ERR_SHAPE.  All calls on one device share that device's array: calls
 * that overlap on one device (other streams, other threads) race and must be
 * serialised by the caller. */
int rq_mlp_swiglu_noalloc(rq_ctx *ctx, const rq_qweight *gate, const rq_qweight *up, const rq_qweight *down,
                          const void *x, rq_dtype x_dtype, void *y, rq_dtype y_dtype, int64_t m, rq_stream stream);

/* Input gradient through a frozen quantized Linear (LoRA fine-tuning):
 * dX[m, k_in] = dY[m, n_out] . deq(W).  The `grad_a = matmul_bt(grad, b)`
 * step of MatMulNode::backward (rusty-autograd/src/lib.rs:152-158) with b the
 * dequantized f32 weight of Linear::forward (rusty-graph/src/lib.rs:69-70);
 * the weight gradient is not formed.  Computed in f32 (one fma per term in
 * ascending n_out, W dequantized exactly as rq_qweight_dequantize does), so
 * with f32 dY and dX the result equals rq_matmul(dY, dequantized W) bit for
 * bit, without materialising the f32 weight.  dy_dtype/dx_dtype: RQ_F32 or
 * RQ_F16. */
int rq_qmatmul_dx(rq_ctx *ctx, const rq_qweight *w, const void *dy, rq_dtype dy_dtype, void *dx, rq_dtype dx_dtype,
                  int64_t m, rq_stream stream);

/* The same input gradient on the matrix cores, for per-row int8 weights (no
 * counterpart in the reference, whose only arithmetic is the f32 chain; for
 * fine-tuning loops that run it every step).  A table built once per weight
 * holds the codes transposed, so that the reduction over n_out is contiguous
 * for the matrix cores, written twice side by side, and k_in unit scales:
 * rq_qweight_dx_table_bytes(w) bytes (0: the weight is not served -- per-row
 * int8 codes, 16-byte aligned, n_out a multiple of 32, k_in of 16),
 * 256-byte aligned, filled by rq_qweight_dx_table.  rq_qmatmul_dx_mfma then
 * forms v = dY . s per row (f32), splits it into two fp16 halves under a
 * per-row power of two (any finite row; hi + lo = v to ~2^-22 relative) and
 * runs the prefill GEMM over both halves against the table: exact products,
 * f32 sums -- the f32 bar against the exact product, not rq_qmatmul_dx's bit
 * pattern.  workspace: rq_qmatmul_dx_mfma_workspace(m, n_out) bytes,
 * 256-byte aligned.  dX fp16 needs 8-byte, f32 16-byte alignment.  Uses the
 * context's GEMM workspace as rq_qmatmul does. */
size_t rq_qweight_dx_table_bytes(const rq_qweight *w);
int rq_qweight_dx_table(rq_ctx *ctx, const rq_qweight *w, void *table, size_t table_bytes, rq_stream stream);
size_t rq_qmatmul_dx_mfma_workspace(int64_t m, int64_t n_out);
int rq_qmatmul_dx_mfma(rq_ctx *ctx, const rq_qweight *w, const void *table, const void *dy, rq_dtype dy_dtype,
                       void *dx, rq_dtype dx_dtype, int64_t m, void *workspace, size_t workspace_bytes,
                       rq_stream stream);

/* ---- int8-weight Llama greedy decode ------------------------------------
 * LlamaModel::forward (rusty-graph/src/lib.rs:420-436) over LlamaBlock
 * (:364-378: norm1 -> Attention -> add -> norm2 -> MLP -> add), Attention
 * with RoPE and a KV cache (:191-283; KVCacheLayer :473-478), RMSNorm
 * (kernels.wgsl:87-102, every row), greedy top_k with k = 1
 * (kernels.wgsl:173-188) and the embedding gather (lib.rs:121-135) on the
 * device.  The reference has no decode loop; this runner defines it: steps
 * are replayed from captured HIP graphs (four steps per launch, see
 * rq_llama_decode), with the position, the token sequence and the KV cache
 * in device memory.  Weights are borrowed (device pointers that must
 * outlive the runner) except q/k/v, which are packed into one [q;k;v] weight
 * owned by the runner at create. */
typedef struct rq_llama_config {
    int32_t n_layers;
    int32_t hidden;       /* = n_heads * head_dim                            */
    int32_t n_heads;
    int32_t n_kv_heads;   /* n_heads % n_kv_heads == 0 (GQA)                  */
    int32_t head_dim;     /* 64 or 128                                        */
    int32_t intermediate;
    int32_t vocab;
    int32_t max_seq;      /* KV cache capacity in tokens, <= 32768            */
    float norm_eps;       /* RMSNorm epsilon (1e-5 in the reference)          */
    float rope_theta;     /* RoPE base (10000 in the reference)               */
} rq_llama_config;

/* One LlamaBlock's weights.  Norm weights are fp16 [hidden]; Linear weights
 * are per-row int8 (RQ_Q_ROWWISE_I8) or the reference's affine u8 codes
 * (RQ_Q_AFFINE_U8, group % 16 == 0 dividing k_in; q/k/v alike in format,
 * group and bias presence, gate/up likewise) in [out, in] orientation:
 * q [n_heads*head_dim, hidden], k/v [n_kv_heads*head_dim, hidden],
 * o [hidden, n_heads*head_dim], gate/up [intermediate, hidden],
 * down [hidden, intermediate]. */
typedef struct rq_llama_layer {
    const void *attn_norm; /* input_layernorm            */
    rq_qweight q, k, v, o;
    const void *mlp_norm;  /* post_attention_layernorm   */
    rq_qweight gate, up, down;
} rq_llama_layer;

typedef struct rq_llama_weights {
    const void *embed;             /* fp16 [vocab, hidden]                 */
    const rq_llama_layer *layers;  /* host array of n_layers               */
    const void *final_norm;        /* fp16 [hidden]                        */
    rq_qweight lm_head;            /* [vocab, hidden], either format       */
} rq_llama_weights;

typedef struct rq_llama rq_llama;

/* Validates the weights against the config, packs q/k/v and allocates the KV
 * cache and step state.  The step graph is captured later, by the first step
 * that runs in graph mode (see rq_llama_decode), so a runner that only steps
 * eagerly never captures one. */
int rq_llama_create(rq_ctx *ctx, const rq_llama_config *cfg, const rq_llama_weights *w, rq_llama **out);
int rq_llama_destroy(rq_llama *model);
/* Starts a sequence: runs the n prompt tokens (host array, each < vocab)
 * through the model, filling the KV cache; the greedy token of the last
 * position becomes token n of the sequence.  By default the prompt runs in
 * batched chunks (every position of a chunk at once: [rows, hidden] GEMMs
 * and a causal prefill attention); see rq_llama_set_prefill.  Uses the
 * context's GEMM workspace when `stream` is the context stream (NULL), so
 * runs on other streams must not overlap other GEMM work of the context.
 * Asynchronous apart from the token upload. */
int rq_llama_prefill(rq_llama *model, const int32_t *tokens, int32_t n, rq_stream stream);
/* Positions per batched prefill chunk: a multiple of 32 up to
 * min(max_seq rounded up to 32, 2048) (the default), or 0 to run the prompt
 * one position at a time through the decode step (the step graph).
 * No reference counterpart (the reference has no prompt loop). */
int rq_llama_set_prefill(rq_llama *model, int32_t rows);
/* n_steps greedy decode steps, each feeding the previous token.  The
 * sequence grows by n_steps; fails with RQ_ERR_SHAPE past max_seq cached
 * positions.  Asynchronous (graph launches only).  In graph mode a run
 * replays a graph of four consecutive steps for each full four and a
 * one-step graph for the rest; the first run that needs either captures and
 * instantiates it on `stream` (stream capture, no device work) before
 * launching it. */
int rq_llama_decode(rq_llama *model, int32_t n_steps, rq_stream stream);
/* Steps run as graph launches (default, use_graph = 1: four steps or one
 * per launch) or as direct kernel launches on the stream (0: for tools that
 * do not trace graphs). */
int rq_llama_set_graph(rq_llama *model, int use_graph);
/* Copies up to `capacity` tokens of the sequence (prompt, then generated) to
 * host memory and stores the sequence length in *length.  Synchronizes. */
int rq_llama_tokens(rq_llama *model, int32_t *out, int32_t capacity, int32_t *length, rq_stream stream);
/* Copies the last step's f32 logits [vocab] to host memory.  Synchronizes. */
int rq_llama_logits(rq_llama *model, float *out, rq_stream stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* RUSTY_HIP_H */
