// C-ABI layer: argument validation, context/stream/memory plumbing and
// dispatch to the gfx950 kernels.  Declarations and the reference interface
// each entry point replaces are in include/rusty_hip.h.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <new>

#include "common.hpp"

namespace rq {

static thread_local char g_err[512];

int fail(int status, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return status;
}

int enter(rq_ctx *ctx) {
    g_err[0] = '\0';
    if (!ctx) return fail(RQ_ERR_INVALID_ARGUMENT, "null context");
    int cur = -1;
    RQ_HIP_TRY(hipGetDevice(&cur));
    if (cur != ctx->device) RQ_HIP_TRY(hipSetDevice(ctx->device));
    return RQ_OK;
}

bool mul_ok(int64_t a, int64_t b, int64_t *out) {
    if (a < 0 || b < 0) return false;
    if (a != 0 && b > INT64_MAX / a) return false;
    *out = a * b;
    return true;
}

}  // namespace rq

using namespace rq;

int rq::check_qweight(const rq_qweight *w) {
    if (!w) return fail(RQ_ERR_INVALID_ARGUMENT, "null weight");
    if (w->format != RQ_Q_ROWWISE_I8 && w->format != RQ_Q_AFFINE_U8)
        return fail(RQ_ERR_INVALID_ARGUMENT, "unknown weight format %d", w->format);
    if (w->n_out < 0 || w->k_in < 0) return fail(RQ_ERR_SHAPE, "negative weight shape");
    int64_t n;
    if (!mul_ok(w->n_out, w->k_in, &n)) return fail(RQ_ERR_SHAPE, "weight shape overflows");
    if (w->format == RQ_Q_AFFINE_U8 && w->group <= 0)
        return fail(RQ_ERR_INVALID_ARGUMENT, "affine weight needs group > 0");
    if (n > 0 && !w->codes) return fail(RQ_ERR_INVALID_ARGUMENT, "null codes");
    if (w->n_out > 0 && !w->scales) return fail(RQ_ERR_INVALID_ARGUMENT, "null scales");
    if (w->prep && (w->format != RQ_Q_AFFINE_U8 || !aligned(w->prep, 16)))
        return fail(RQ_ERR_INVALID_ARGUMENT, "a prepared table belongs to an affine weight and is 16-byte aligned");
    return RQ_OK;
}

// One wave waits on the device's constant-rate wall clock (wall_clock64,
// `ticks` periods) and exits; s_sleep between reads keeps the wave idle.
__global__ void k_device_delay(uint64_t ticks) {
    const uint64_t t0 = wall_clock64();
    while (wall_clock64() - t0 < ticks) __builtin_amdgcn_s_sleep(32);
}

// One lane stores the device's constant-rate wall clock when the stream
// reaches this launch.
__global__ void k_device_clock(uint64_t *dst) {
    if (threadIdx.x == 0) *dst = wall_clock64();
}

// Measurement aid: the weight stream of the decode GEMV without its
// arithmetic.  Block b reads rows [b*R, b*R + R) of `rows` rows of row_bytes
// bytes; thread t reads 16-byte chunks t, t + 256, ... (CPT of them) of each
// row with the non-temporal policy, like the GEMV's weight loads (all in
// flight, then combined).  Each wave XOR-reduces its lanes' words with DPP
// steps, so every lane's loads feed the result; with store, lane 0 of wave
// r < R stores it (folded to 2 bytes) for row b*R + r, as the GEMV stores its
// fp16 output; without, it is stored only if it equals an all-ones word (never,
// in practice), so the loads stay live and nothing is written.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}
template <int R, int CPT>
__global__ __launch_bounds__(256) void k_stream_probe(const uint8_t *__restrict__ src, int row_bytes, int rows,
                                                      uint16_t *__restrict__ dst, int store) {
    typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int row0 = blockIdx.x * R, rows_here = min(R, rows - row0);
    const auto rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(src) + (size_t)row0 * row_bytes, 0,
                                                      (uint32_t)(rows_here * row_bytes), 0x00020000);
    const int C = row_bytes / 16;
    u32x4 v[R][CPT];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int j = 0; j < CPT; ++j) {
            const int c = t + 256 * j;  // rows past the resource read as zero
            v[r][j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                    rs, c < C ? (uint32_t)(r * row_bytes + c * 16) : 0x80000000u, 0, 2));
        }
    uint32_t acc = 0;
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int j = 0; j < CPT; ++j) acc ^= v[r][j].x ^ v[r][j].y ^ v[r][j].z ^ v[r][j].w;
    acc ^= dpp_u32<0xB1>(acc);   // quad_perm [1,0,3,2]
    acc ^= dpp_u32<0x4E>(acc);   // quad_perm [2,3,0,1]
    acc ^= dpp_u32<0x141>(acc);  // row_half_mirror
    acc ^= dpp_u32<0x140>(acc);  // row_mirror: each 16-lane row holds its XOR
    acc = (uint32_t)__builtin_amdgcn_readlane((int)acc, 0) ^ (uint32_t)__builtin_amdgcn_readlane((int)acc, 16) ^
          (uint32_t)__builtin_amdgcn_readlane((int)acc, 32) ^ (uint32_t)__builtin_amdgcn_readlane((int)acc, 48);
    if (lane == 0 && wave < rows_here && (store || acc == 0xFFFFFFFFu)) dst[row0 + wave] = (uint16_t)(acc ^ (acc >> 16));
}

template <int R>
void launch_probe(int cpt, unsigned blocks, hipStream_t s, const uint8_t *src, int row_bytes, int rows, uint16_t *dst,
                  int store) {
    switch (cpt) {
    case 1: hipLaunchKernelGGL((k_stream_probe<R, 1>), dim3(blocks), dim3(256), 0, s, src, row_bytes, rows, dst, store); break;
    case 2: hipLaunchKernelGGL((k_stream_probe<R, 2>), dim3(blocks), dim3(256), 0, s, src, row_bytes, rows, dst, store); break;
    case 3: hipLaunchKernelGGL((k_stream_probe<R, 3>), dim3(blocks), dim3(256), 0, s, src, row_bytes, rows, dst, store); break;
    default: hipLaunchKernelGGL((k_stream_probe<R, 4>), dim3(blocks), dim3(256), 0, s, src, row_bytes, rows, dst, store); break;
    }
}

// One wave, `steps` dependent f32 fmas per lane (acc = fma(acc, a, b), a and
// b kernel arguments so nothing folds), the result stored: the latency of a
// k-ascending fma chain, which bounds the f32 matmul's chain kernels where
// few outputs each walk a long k.
__global__ __launch_bounds__(64) void k_fma_chain_probe(float a, float b, int64_t steps, float *__restrict__ dst) {
    float acc = (float)threadIdx.x;
    int64_t i = 0;
    for (; i + 16 <= steps; i += 16) {
#pragma unroll
        for (int u = 0; u < 16; ++u) acc = __builtin_fmaf(acc, a, b);
    }
    for (; i < steps; ++i) acc = __builtin_fmaf(acc, a, b);
    dst[threadIdx.x] = acc;
}

// Byte fill: 16-byte stores over the aligned middle (grid-stride), single
// bytes for the unaligned head and tail.  A kernel rather than
// hipMemsetAsync, so that a caller may capture it in a HIP graph: memset
// nodes in captured graphs have given wrong results on replays here.
__global__ __launch_bounds__(256) void k_fill_bytes(uint8_t *__restrict__ dst, uint32_t v4, size_t head, size_t chunks,
                                                   size_t n) {
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x, stride = (size_t)gridDim.x * blockDim.x;
    const uint4 v = make_uint4(v4, v4, v4, v4);
    uint4 *mid = reinterpret_cast<uint4 *>(dst + head);
    for (size_t i = t; i < chunks; i += stride) mid[i] = v;
    const size_t tail0 = head + chunks * 16;
    if (t < head) dst[t] = (uint8_t)v4;
    if (t < n - tail0) dst[tail0 + t] = (uint8_t)v4;
}

extern "C" {

const char *rq_status_string(int status) {
    switch (status) {
    case RQ_OK: return "RQ_OK";
    case RQ_ERR_INVALID_ARGUMENT: return "RQ_ERR_INVALID_ARGUMENT";
    case RQ_ERR_SHAPE: return "RQ_ERR_SHAPE";
    case RQ_ERR_UNSUPPORTED: return "RQ_ERR_UNSUPPORTED";
    case RQ_ERR_HIP: return "RQ_ERR_HIP";
    case RQ_ERR_NO_DEVICE: return "RQ_ERR_NO_DEVICE";
    case RQ_ERR_ALLOC: return "RQ_ERR_ALLOC";
    default: return "RQ_ERR_UNKNOWN";
    }
}

const char *rq_last_error(void) { return g_err; }

int rq_ctx_create(int device, rq_ctx **out) {
    g_err[0] = '\0';
    if (!out) return fail(RQ_ERR_INVALID_ARGUMENT, "null output pointer");
    *out = nullptr;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= 0)
        return fail(RQ_ERR_NO_DEVICE, "no HIP device visible");
    if (device < 0 || device >= count)
        return fail(RQ_ERR_NO_DEVICE, "device %d out of range (%d visible)", device, count);
    hipDeviceProp_t prop;
    RQ_HIP_TRY(hipGetDeviceProperties(&prop, device));
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(RQ_ERR_NO_DEVICE, "device %d is %s; this library is built for gfx950 only", device,
                    prop.gcnArchName);
    RQ_HIP_TRY(hipSetDevice(device));
    rq_ctx *ctx = new (std::nothrow) rq_ctx;
    if (!ctx) return fail(RQ_ERR_ALLOC, "context allocation failed");
    ctx->device = device;
    ctx->num_cus = prop.multiProcessorCount;
    ctx->sk_partials = nullptr;
    ctx->sk_counters = nullptr;
    ctx->prep = nullptr;
    // Default priority on purpose: streams of mixed priorities are not used.
    hipError_t e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        delete ctx;
        return fail(RQ_ERR_HIP, "hipStreamCreateWithFlags: %s", hipGetErrorString(e));
    }
    // Split-K workspace of the prefill GEMM (32 MiB of partial sums, 512 KiB
    // of counters that must start at zero).  Without it the GEMM never splits.
    {
        const size_t part = kGemmSkFloats * 4, cnt = (size_t)kGemmSkCounters * 128;
        void *p = nullptr;
        if (hipMalloc(&p, part + cnt) == hipSuccess) {
            if (hipMemset(static_cast<char *>(p) + part, 0, cnt) == hipSuccess && hipDeviceSynchronize() == hipSuccess) {
                ctx->sk_partials = static_cast<float *>(p);
                ctx->sk_counters = reinterpret_cast<int *>(static_cast<char *>(p) + part);
            } else {
                (void)hipFree(p);
            }
        }
        (void)hipGetLastError();  // a failed optional allocation is not the caller's error
    }
    // Input preparation of the prefill GEMM for affine weights and f32
    // activations; without it those requests take the generic kernel.
    {
        void *p = nullptr;
        if (hipMalloc(&p, kGemmPrepBytes) == hipSuccess) ctx->prep = p;
        (void)hipGetLastError();
    }
    noalloc_init(device);  // the no-alloc SwiGLU's scratch address on this device
    *out = ctx;
    return RQ_OK;
}

int rq_ctx_destroy(rq_ctx *ctx) {
    if (!ctx) return RQ_OK;
    RQ_ENTER(ctx);
    hipError_t e1 = hipStreamSynchronize(ctx->stream);
    hipError_t e2 = hipStreamDestroy(ctx->stream);
    if (ctx->sk_partials) (void)hipFree(ctx->sk_partials);
    if (ctx->prep) (void)hipFree(ctx->prep);
    delete ctx;
    if (e1 != hipSuccess) return fail(RQ_ERR_HIP, "hipStreamSynchronize: %s", hipGetErrorString(e1));
    if (e2 != hipSuccess) return fail(RQ_ERR_HIP, "hipStreamDestroy: %s", hipGetErrorString(e2));
    return RQ_OK;
}

int rq_ctx_stream(rq_ctx *ctx, rq_stream *out) {
    RQ_ENTER(ctx);
    if (!out) return fail(RQ_ERR_INVALID_ARGUMENT, "null output pointer");
    *out = ctx->stream;
    return RQ_OK;
}

int rq_ctx_num_cus(rq_ctx *ctx, int *out) {
    RQ_ENTER(ctx);
    if (!out) return fail(RQ_ERR_INVALID_ARGUMENT, "null output pointer");
    *out = ctx->num_cus;
    return RQ_OK;
}

int rq_sync(rq_ctx *ctx, rq_stream stream) {
    RQ_ENTER(ctx);
    RQ_HIP_TRY(hipStreamSynchronize(pick(ctx, stream)));
    return RQ_OK;
}

int rq_device_delay(rq_ctx *ctx, uint32_t microseconds, rq_stream stream) {
    RQ_ENTER(ctx);
    if (microseconds > 100000u) return fail(RQ_ERR_INVALID_ARGUMENT, "delay of %u us is above 100000 us", microseconds);
    if (microseconds == 0) return RQ_OK;
    int khz = 0;  // wall clock rate in kHz (100 MHz on gfx9)
    if (hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, ctx->device) != hipSuccess || khz <= 0) khz = 100000;
    const uint64_t ticks = (uint64_t)microseconds * (uint64_t)khz / 1000u;
    hipLaunchKernelGGL(k_device_delay, dim3(1), dim3(64), 0, pick(ctx, stream), ticks);
    RQ_LAUNCH_CHECK();
    return RQ_OK;
}

int rq_device_clock(rq_ctx *ctx, uint64_t *dst, uint64_t *ticks_per_second, rq_stream stream) {
    RQ_ENTER(ctx);
    if (!dst) return fail(RQ_ERR_INVALID_ARGUMENT, "null destination");
    if (ticks_per_second) {
        int khz = 0;
        RQ_HIP_TRY(hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, ctx->device));
        if (khz <= 0) return fail(RQ_ERR_HIP, "device reports no wall clock rate");
        *ticks_per_second = (uint64_t)khz * 1000u;
    }
    hipLaunchKernelGGL(k_device_clock, dim3(1), dim3(64), 0, pick(ctx, stream), dst);
    RQ_LAUNCH_CHECK();
    return RQ_OK;
}

int rq_fma_chain_probe(rq_ctx *ctx, int64_t steps, float *dst, rq_stream stream) {
    RQ_ENTER(ctx);
    if (!dst) return fail(RQ_ERR_INVALID_ARGUMENT, "null pointer");
    if (steps < 0) return fail(RQ_ERR_SHAPE, "negative step count");
    hipLaunchKernelGGL(k_fma_chain_probe, dim3(1), dim3(64), 0, pick(ctx, stream), 1.0000001f, 1e-7f, steps, dst);
    RQ_LAUNCH_CHECK();
    return RQ_OK;
}

int rq_stream_probe(rq_ctx *ctx, const void *src, size_t row_bytes, size_t rows, int rows_per_block, void *dst,
                    int store, rq_stream stream) {
    RQ_ENTER(ctx);
    if (rows == 0) return RQ_OK;
    if (!src || !dst) return fail(RQ_ERR_INVALID_ARGUMENT, "null pointer");
    if (row_bytes == 0 || row_bytes % 16 != 0 || row_bytes > 16384)
        return fail(RQ_ERR_SHAPE, "row_bytes must be a multiple of 16 in 16..16384");
    if (rows_per_block < 1 || rows_per_block > 4) return fail(RQ_ERR_SHAPE, "rows_per_block must be 1..4");
    if (rows > 0x7fffffff || rows * row_bytes > 0xffffffffull) return fail(RQ_ERR_SHAPE, "too many rows");
    if (!aligned(src, 16) || !aligned(dst, 2)) return fail(RQ_ERR_INVALID_ARGUMENT, "misaligned pointer");
    const unsigned blocks = (unsigned)cdiv((int64_t)rows, rows_per_block);
    const int cpt = (int)cdiv((int64_t)row_bytes / 16, 256);
    const auto *sp = static_cast<const uint8_t *>(src);
    auto *dp = static_cast<uint16_t *>(dst);
    hipStream_t s = pick(ctx, stream);
    const int st = store ? 1 : 0;
    if (rows_per_block == 1) launch_probe<1>(cpt, blocks, s, sp, (int)row_bytes, (int)rows, dp, st);
    else if (rows_per_block == 2) launch_probe<2>(cpt, blocks, s, sp, (int)row_bytes, (int)rows, dp, st);
    else if (rows_per_block == 3) launch_probe<3>(cpt, blocks, s, sp, (int)row_bytes, (int)rows, dp, st);
    else launch_probe<4>(cpt, blocks, s, sp, (int)row_bytes, (int)rows, dp, st);
    RQ_LAUNCH_CHECK();
    return RQ_OK;
}

int rq_alloc(rq_ctx *ctx, size_t bytes, void **dptr) {
    RQ_ENTER(ctx);
    if (!dptr) return fail(RQ_ERR_INVALID_ARGUMENT, "null output pointer");
    *dptr = nullptr;
    if (bytes == 0) return RQ_OK;
    hipError_t e = hipMalloc(dptr, bytes);
    if (e != hipSuccess) {
        *dptr = nullptr;
        return fail(RQ_ERR_ALLOC, "hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
    }
    return RQ_OK;
}

int rq_free(rq_ctx *ctx, void *dptr) {
    RQ_ENTER(ctx);
    if (!dptr) return RQ_OK;
    RQ_HIP_TRY(hipFree(dptr));
    return RQ_OK;
}

static int copy(rq_ctx *ctx, void *dst, const void *src, size_t bytes, hipMemcpyKind kind, rq_stream stream) {
    RQ_ENTER(ctx);
    if (bytes == 0) return RQ_OK;
    if (!dst || !src) return fail(RQ_ERR_INVALID_ARGUMENT, "null pointer in copy");
    hipStream_t s = pick(ctx, stream);
    RQ_HIP_TRY(hipMemcpyAsync(dst, src, bytes, kind, s));
    // Host buffers are pageable and owned by the caller: complete the copy
    // before returning, as UnifiedTensor::new / to_vec do.
    if (kind != hipMemcpyDeviceToDevice) RQ_HIP_TRY(hipStreamSynchronize(s));
    return RQ_OK;
}

int rq_memcpy_h2d(rq_ctx *ctx, void *dst, const void *src, size_t bytes, rq_stream stream) {
    return copy(ctx, dst, src, bytes, hipMemcpyHostToDevice, stream);
}
int rq_memcpy_d2h(rq_ctx *ctx, void *dst, const void *src, size_t bytes, rq_stream stream) {
    return copy(ctx, dst, src, bytes, hipMemcpyDeviceToHost, stream);
}
int rq_memcpy_d2d(rq_ctx *ctx, void *dst, const void *src, size_t bytes, rq_stream stream) {
    return copy(ctx, dst, src, bytes, hipMemcpyDeviceToDevice, stream);
}

int rq_memset(rq_ctx *ctx, void *dst, int value, size_t bytes, rq_stream stream) {
    RQ_ENTER(ctx);
    if (bytes == 0) return RQ_OK;
    if (!dst) return fail(RQ_ERR_INVALID_ARGUMENT, "null pointer in memset");
    const uint32_t b = (uint32_t)(value & 0xff), v4 = b * 0x01010101u;
    const size_t mis = reinterpret_cast<uintptr_t>(dst) % 16, head = mis ? std::min(bytes, 16 - mis) : 0;
    const size_t chunks = (bytes - head) / 16;  // the tail (< 16 bytes) is what remains
    const size_t blocks = std::min<size_t>(std::max<size_t>(cdiv((int64_t)chunks, 256), 1), 4096);
    hipLaunchKernelGGL(k_fill_bytes, dim3((unsigned)blocks), dim3(256), 0, pick(ctx, stream), static_cast<uint8_t *>(dst),
                       v4, head, chunks, bytes);
    RQ_LAUNCH_CHECK();
    return RQ_OK;
}

int rq_dequantize(rq_ctx *ctx, const uint32_t *input, size_t n_words, float *out, size_t n_out,
                  rq_stream stream) {
    RQ_ENTER(ctx);
    if (n_words == 0 || n_out == 0) return RQ_OK;
    if (!input || !out) return fail(RQ_ERR_INVALID_ARGUMENT, "null pointer");
    if (n_words > SIZE_MAX / 4) return fail(RQ_ERR_SHAPE, "n_words too large");
    return launch_dequantize(input, n_words, out, n_out, pick(ctx, stream));
}

int rq_affine_dequantize(rq_ctx *ctx, const uint32_t *weight, size_t n_weight_words, const float *scales,
                         const float *biases, size_t n_groups, float *out, size_t n_out, uint32_t group,
                         uint32_t flags, rq_stream stream) {
    RQ_ENTER(ctx);
    if (flags & ~RQ_AFFINE_FMA) return fail(RQ_ERR_INVALID_ARGUMENT, "unknown flags 0x%x", flags);
    if (group == 0) return fail(RQ_ERR_INVALID_ARGUMENT, "group must be > 0");
    if (n_out == 0) return RQ_OK;
    if (!weight || !scales || !out) return fail(RQ_ERR_INVALID_ARGUMENT, "null pointer");
    if (n_weight_words < (n_out + 3) / 4)
        return fail(RQ_ERR_SHAPE, "weight has %zu words, %zu elements need %zu", n_weight_words, n_out,
                    (n_out + 3) / 4);
    if (n_groups < (n_out + group - 1) / group)
        return fail(RQ_ERR_SHAPE, "%zu scale groups, %zu elements need %zu", n_groups, n_out,
                    (n_out + group - 1) / group);
    return launch_affine_dequantize(weight, scales, biases, out, n_out, group, (flags & RQ_AFFINE_FMA) != 0,
                                    pick(ctx, stream));
}


int rq_qweight_dequantize(rq_ctx *ctx, const rq_qweight *w, float *out, rq_stream stream) {
    RQ_ENTER(ctx);
    int st = check_qweight(w);
    if (st != RQ_OK) return st;
    const size_t n = (size_t)w->n_out * (size_t)w->k_in;
    if (n == 0) return RQ_OK;
    if (!out) return fail(RQ_ERR_INVALID_ARGUMENT, "null output");
    if (w->format == RQ_Q_ROWWISE_I8)
        return launch_rowwise_dequantize((const int8_t *)w->codes, w->scales, out, w->n_out, w->k_in,
                                         pick(ctx, stream));
    // The affine kernel reads the codes as u32 words; a byte count that is
    // not a multiple of 4 would make its last word read past the buffer, so
    // such tails take the byte path inside the kernel (n bounds every read).
    return launch_affine_dequantize((const uint32_t *)w->codes, w->scales, w->biases, out, n, (uint32_t)w->group,
                                    false, pick(ctx, stream));
}

size_t rq_qweight_prep_bytes(const rq_qweight *w) {
    if (!w || check_qweight(w) != RQ_OK) return 0;
    return affine_prep_bytes(*w);
}

int rq_qweight_prepare(rq_ctx *ctx, rq_qweight *w, void *table, size_t table_bytes, rq_stream stream) {
    RQ_ENTER(ctx);
    if (!w) return fail(RQ_ERR_INVALID_ARGUMENT, "null weight");
    w->prep = nullptr;
    int st = check_qweight(w);
    if (st != RQ_OK) return st;
    const size_t need = affine_prep_bytes(*w);
    if (need == 0) return RQ_OK;  // nothing the GEMM would read
    if (!table) return fail(RQ_ERR_INVALID_ARGUMENT, "null table");
    if (!aligned(table, 16)) return fail(RQ_ERR_INVALID_ARGUMENT, "table must be 16-byte aligned");
    if (table_bytes < need) return fail(RQ_ERR_SHAPE, "table of %zu bytes, the weight needs %zu", table_bytes, need);
    if ((st = launch_affine_prep(*w, static_cast<float *>(table), pick(ctx, stream))) != RQ_OK) return st;
    w->prep = static_cast<const float *>(table);
    return RQ_OK;
}

static int matmul_common(rq_ctx *ctx, int variant, const float *a, const float *b, float *out, int64_t m,
                         int64_t k, int64_t n, rq_stream stream) {
    RQ_ENTER(ctx);
    if (m < 0 || k < 0 || n < 0) return fail(RQ_ERR_SHAPE, "negative matmul shape");
    int64_t t;
    if (!mul_ok(m, k, &t) || !mul_ok(k, n, &t) || !mul_ok(m, n, &t)) return fail(RQ_ERR_SHAPE, "shape overflows");
    if (m == 0 || n == 0) return RQ_OK;
    if (!out || (k > 0 && (!a || !b))) return fail(RQ_ERR_INVALID_ARGUMENT, "null pointer");
    return launch_matmul_f32(variant, a, b, out, m, k, n, pick(ctx, stream));
}

int rq_matmul(rq_ctx *ctx, const float *a, const float *b, float *out, int64_t m, int64_t k, int64_t n,
              rq_stream stream) {
    return matmul_common(ctx, MM_AB, a, b, out, m, k, n, stream);
}
int rq_matmul_bt(rq_ctx *ctx, const float *a, const float *b, float *out, int64_t m, int64_t k, int64_t n,
                 rq_stream stream) {
    return matmul_common(ctx, MM_ABT, a, b, out, m, k, n, stream);
}
int rq_matmul_at(rq_ctx *ctx, const float *a, const float *b, float *out, int64_t m, int64_t k, int64_t n,
                 rq_stream stream) {
    return matmul_common(ctx, MM_ATB, a, b, out, m, k, n, stream);
}

}  // extern "C"

rq::GemmWorkspace rq::gemm_workspace(const rq_ctx *ctx, hipStream_t s) {
    GemmWorkspace ws{nullptr, nullptr, 0, 0};
    if (s != ctx->stream) return ws;
    if (ctx->sk_partials) ws = GemmWorkspace{ctx->sk_partials, ctx->sk_counters, kGemmSkFloats, kGemmSkCounters};
    if (ctx->prep) {
        ws.prep = ctx->prep;
        ws.prep_bytes = kGemmPrepBytes;
    }
    return ws;
}

// Fused linear dispatch (arguments already validated): decode kernels for
// few tokens, the MFMA GEMM for many, the generic kernel for anything the
// tuned paths do not serve.
int rq::qmatmul_dispatch(rq_ctx *ctx, const rq_qweight &w, const void *x, rq_dtype xt, void *y, rq_dtype yt,
                         int64_t m, const GemmWorkspace &ws, hipStream_t s) {
    if (w.k_in > 0) {
        // 1-2 tokens: the VALU dot2 GEMV; 3-16: the MFMA GEMV (measured faster
        // from 3 tokens on, e.g. 4096x4096 m = 4: 7.2 -> 6.3 us); the VALU
        // kernel also serves the 3-4 token shapes the MFMA kernel refuses
        // (affine codes).
        int st = RQ_ERR_UNSUPPORTED;
        // f32 activations take the same kernels, each value carried as two
        // fp16 terms after a power-of-two scaling that keeps it in range
        if (m <= 2) st = launch_gemv_decode(w, x, xt, y, yt, (int)m, s);
        if (st == RQ_ERR_UNSUPPORTED && m <= 16) st = launch_gemv_mfma(w, x, xt, y, yt, (int)m, s);
        if (st == RQ_ERR_UNSUPPORTED && m <= 4 && xt == RQ_F16) st = launch_gemv_decode(w, x, xt, y, yt, (int)m, s);
        if (st == RQ_ERR_UNSUPPORTED && m <= 8) st = launch_gemv(w, x, xt, y, yt, (int)m, ctx->num_cus, s);
        if (st == RQ_ERR_UNSUPPORTED) st = launch_gemm(w, x, xt, y, yt, m, ctx->num_cus, ws, s);
        if (st != RQ_ERR_UNSUPPORTED) return st;
    }
    return launch_qlinear_generic(w, x, xt, y, yt, m, s);
}

// Argument checks shared by rq_mlp_swiglu and its no-alloc variant (pointers
// are checked by the callers).
int rq::swiglu_check(const rq_qweight *gate, const rq_qweight *up, const rq_qweight *down, rq_dtype x_dtype,
                     rq_dtype y_dtype, int64_t m) {
    int st;
    if ((st = check_qweight(gate)) != RQ_OK || (st = check_qweight(up)) != RQ_OK || (st = check_qweight(down)) != RQ_OK)
        return st;
    if ((x_dtype != RQ_F16 && x_dtype != RQ_F32) || (y_dtype != RQ_F16 && y_dtype != RQ_F32))
        return fail(RQ_ERR_INVALID_ARGUMENT, "dtype must be RQ_F16 or RQ_F32");
    const int64_t I = gate->n_out, H = gate->k_in;
    if (up->n_out != I || up->k_in != H || down->n_out != H || down->k_in != I)
        return fail(RQ_ERR_SHAPE, "SwiGLU shapes: gate/up [%lld,%lld], down must be [%lld,%lld]", (long long)I,
                    (long long)H, (long long)H, (long long)I);
    if (m < 0) return fail(RQ_ERR_SHAPE, "negative m");
    int64_t t;
    if (!mul_ok(m, 2 * I, &t) || !mul_ok(m, H, &t)) return fail(RQ_ERR_SHAPE, "shape overflows");
    return RQ_OK;
}

// The SwiGLU MLP over validated arguments, h a workspace of 2*m*I fp16 values:
// the gate/up pass writes h = silu(g) * u into its first m*I values (the
// prefill fallback stages g and u in its two halves first), then the down
// projection reads it.  ws: the split-K workspace the prefill GEMMs may use.
int rq::swiglu_run(rq_ctx *ctx, const rq_qweight &gate, const rq_qweight &up, const rq_qweight &down, const void *x,
                   rq_dtype x_dtype, void *h, void *y, rq_dtype y_dtype, int64_t m, const GemmWorkspace &ws,
                   hipStream_t s) {
    const int64_t I = gate.n_out;
    // no intermediate features: h is empty and the down projection's
    // reduction too (y = 0)
    if (I == 0) return qmatmul_dispatch(ctx, down, h, RQ_F16, y, y_dtype, m, ws, s);
    int st = RQ_ERR_UNSUPPORTED;
    if (m <= 2) st = launch_swiglu_decode(gate, up, x, x_dtype, h, (int)m, s);
    if (st == RQ_ERR_UNSUPPORTED && m <= 16) st = launch_swiglu_mfma(gate, up, x, x_dtype, h, (int)m, s);
    if (st == RQ_ERR_UNSUPPORTED && x_dtype == RQ_F16 && m <= 4)
        st = launch_swiglu_decode(gate, up, x, x_dtype, h, (int)m, s);
    if (st == RQ_ERR_UNSUPPORTED && m > 16) {
        // prefill: gate and up in one GEMM launch with the silu*mul epilogue
        // where it serves them; else two GEMMs into the two halves of the
        // workspace, then h = silu(g) * u in place over the first half
        st = launch_gemm_swiglu(gate, up, x, x_dtype, h, m, ctx->num_cus, ws, s);
        if (st == RQ_ERR_UNSUPPORTED) {
            _Float16 *g = static_cast<_Float16 *>(h), *u = g + m * I;
            st = launch_gemm(gate, x, x_dtype, g, RQ_F16, m, ctx->num_cus, ws, s);
            if (st == RQ_OK) st = launch_gemm(up, x, x_dtype, u, RQ_F16, m, ctx->num_cus, ws, s);
            if (st == RQ_OK) st = launch_silu_mul(g, u, g, m * I, s);
        }
    }
    if (st == RQ_ERR_UNSUPPORTED) st = launch_swiglu_generic(gate, up, x, x_dtype, h, m, s);
    if (st != RQ_OK) return st;
    // down projection of h, with the same workspace
    return qmatmul_dispatch(ctx, down, h, RQ_F16, y, y_dtype, m, ws, s);
}

extern "C" {

int rq_qmatmul(rq_ctx *ctx, const rq_qweight *w, const void *x, rq_dtype x_dtype, void *y, rq_dtype y_dtype,
               int64_t m, rq_stream stream) {
    RQ_ENTER(ctx);
    int st = check_qweight(w);
    if (st != RQ_OK) return st;
    if ((x_dtype != RQ_F16 && x_dtype != RQ_F32) || (y_dtype != RQ_F16 && y_dtype != RQ_F32))
        return fail(RQ_ERR_INVALID_ARGUMENT, "dtype must be RQ_F16 or RQ_F32");
    if (m < 0) return fail(RQ_ERR_SHAPE, "negative m");
    int64_t t;
    if (!mul_ok(m, w->k_in, &t) || !mul_ok(m, w->n_out, &t)) return fail(RQ_ERR_SHAPE, "shape overflows");
    if (m == 0 || w->n_out == 0) return RQ_OK;
    if (!y || (w->k_in > 0 && !x)) return fail(RQ_ERR_INVALID_ARGUMENT, "null activation pointer");
    hipStream_t s = pick(ctx, stream);
    return qmatmul_dispatch(ctx, *w, x, x_dtype, y, y_dtype, m, gemm_workspace(ctx, s), s);
}

int rq_mlp_swiglu(rq_ctx *ctx, const rq_qweight *gate, const rq_qweight *up, const rq_qweight *down, const void *x,
                  rq_dtype x_dtype, void *h, void *y, rq_dtype y_dtype, int64_t m, rq_stream stream) {
    RQ_ENTER(ctx);
    int st = swiglu_check(gate, up, down, x_dtype, y_dtype, m);
    if (st != RQ_OK || m == 0 || gate->k_in == 0) return st;
    // (no intermediate features: h holds nothing and may be null)
    if (!y || (gate->n_out > 0 && !h) || !x) return fail(RQ_ERR_INVALID_ARGUMENT, "null activation or workspace pointer");
    hipStream_t s = pick(ctx, stream);
    return swiglu_run(ctx, *gate, *up, *down, x, x_dtype, h, y, y_dtype, m, gemm_workspace(ctx, s), s);
}

int rq_qmatmul_dx(rq_ctx *ctx, const rq_qweight *w, const void *dy, rq_dtype dy_dtype, void *dx, rq_dtype dx_dtype,
                  int64_t m, rq_stream stream) {
    RQ_ENTER(ctx);
    int st = check_qweight(w);
    if (st != RQ_OK) return st;
    if ((dy_dtype != RQ_F16 && dy_dtype != RQ_F32) || (dx_dtype != RQ_F16 && dx_dtype != RQ_F32))
        return fail(RQ_ERR_INVALID_ARGUMENT, "dtype must be RQ_F16 or RQ_F32");
    if (m < 0) return fail(RQ_ERR_SHAPE, "negative m");
    int64_t t;
    if (!mul_ok(m, w->k_in, &t) || !mul_ok(m, w->n_out, &t)) return fail(RQ_ERR_SHAPE, "shape overflows");
    if (m == 0 || w->k_in == 0) return RQ_OK;
    if (!dx || (w->n_out > 0 && !dy)) return fail(RQ_ERR_INVALID_ARGUMENT, "null gradient pointer");
    return launch_qmatmul_dx(*w, dy, dy_dtype, dx, dx_dtype, m, pick(ctx, stream));
}

}  // extern "C"
