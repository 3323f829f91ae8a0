// Standalone dequantization kernels for gfx950.
//
//   k_dequantize         <- rusty-backend/src/kernels.wgsl:153-166 (`dequantize`)
//   k_affine_dequantize  <- rusty-backend/src/kernels.wgsl:379-400 (`affine_dequantize`)
//   k_rowwise_dequantize    per-row signed int8: f32(q) * scale[row]
//
// All three are HBM-bound byte expansions (1 B in, 4 B out per element, plus
// the group scalars), written so that every wave-wide store is 1 KiB
// contiguous: a wave step covers 1024 elements, lane l loading the 4-byte
// words l, l + 64, l + 128, l + 192 of the step's codes (256 B per load
// instruction) and storing each as a float4 at elements 4 l + 256 j (1 KiB
// per store instruction).  With each thread owning 16 consecutive elements
// instead, every store instruction wrote 16-byte pieces 64 bytes apart
// (4096^2 elements: 27.7 us, 3.0 TB/s; now 12.8 us with the stores below).
// The WGSL runs one invocation per element and re-reads the containing u32
// four times.  The last partial step (or unaligned pointers) takes a
// per-element path with the same arithmetic.
#include "common.hpp"

namespace rq {
namespace {

constexpr int kThreads = 256;
constexpr size_t kMaxBlocks = 1u << 20;

// Byte i of the little-endian u32 word stream, read as a single byte so a
// tail never touches memory past byte n-1.
__device__ __forceinline__ uint32_t byte_at(const uint32_t *words, size_t i) {
    return reinterpret_cast<const uint8_t *>(words)[i];
}

__device__ __forceinline__ float4 bytes_to_f32x4(uint32_t w) {
    return make_float4((float)(w & 0xFFu), (float)((w >> 8) & 0xFFu), (float)((w >> 16) & 0xFFu),
                       (float)(w >> 24));
}

constexpr size_t kStep = 1024;  // elements per wave step

// A float4 store with the non-temporal policy: the output (4 B per element,
// 64 MiB at 4096^2) is written once and not read by this launch; it streams
// past the caches (4096^2 dequantize: 16.8 us with the default policy, 12.8
// with this one -- 6.5 TB/s).
typedef float f32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void st4(float *p, float4 v) {
    const f32x4 e = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(e, reinterpret_cast<f32x4 *>(p));
}

// The wave-step loop: for every full step of 1024 elements below n_full,
// f(words of the step, element index of the step, lane).
template <class F>
__device__ __forceinline__ void wave_steps(size_t n_full, F &&f) {
    const int lane = threadIdx.x & 63;
    const size_t wave = ((size_t)blockIdx.x * kThreads + threadIdx.x) >> 6;
    const size_t n_waves = (size_t)gridDim.x * (kThreads / 64);
    for (size_t st = wave; st < n_full / kStep; st += n_waves) f(st * kStep, lane);
}
__device__ __forceinline__ size_t thread_id() { return (size_t)blockIdx.x * kThreads + threadIdx.x; }
__device__ __forceinline__ size_t n_threads() { return (size_t)gridDim.x * kThreads; }

template <bool VEC>
__global__ __launch_bounds__(kThreads) void k_dequantize(const uint32_t *__restrict__ in,
                                                         float *__restrict__ out, size_t n) {
    const size_t n_full = VEC ? n / kStep * kStep : 0;
    wave_steps(n_full, [&](size_t e0, int lane) {
        const uint32_t *w = in + e0 / 4;
        uint32_t d[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) d[j] = w[64 * j + lane];
#pragma unroll
        for (int j = 0; j < 4; ++j) st4(out + e0 + 256 * j + 4 * lane, bytes_to_f32x4(d[j]));
    });
    for (size_t i = n_full + thread_id(); i < n; i += n_threads()) out[i] = (float)byte_at(in, i);
}

// out = u*s + b.  FMA=false: the multiply and the add each round to f32,
// exactly as `val_u8 * scale + bias` reads in kernels.wgsl:399 without
// contraction.  FMA=true: one rounding.
template <bool FMA>
__device__ __forceinline__ float affine(float u, float s, float b) {
    if constexpr (FMA) {
        return __builtin_fmaf(u, s, b);
    } else {
#pragma clang fp contract(off)
        const float p = u * s;
        return p + b;
    }
}

template <bool FMA>
__device__ __forceinline__ float4 affine4(uint32_t w, float s, float b) {
    return make_float4(affine<FMA>((float)(w & 0xFFu), s, b), affine<FMA>((float)((w >> 8) & 0xFFu), s, b),
                       affine<FMA>((float)((w >> 16) & 0xFFu), s, b), affine<FMA>((float)(w >> 24), s, b));
}

// VEC requires 16-byte aligned pointers and group % 16 == 0 (a lane's 4
// elements then lie in one group); gshift >= 0: group = 1 << gshift.
template <bool VEC, bool FMA>
__global__ __launch_bounds__(kThreads) void k_affine_dequantize(const uint32_t *__restrict__ in,
                                                                const float *__restrict__ scales,
                                                                const float *__restrict__ biases,
                                                                float *__restrict__ out, size_t n,
                                                                uint32_t group, int gshift) {
    const size_t n_full = VEC ? n / kStep * kStep : 0;
    wave_steps(n_full, [&](size_t e0, int lane) {
        const uint32_t *w = in + e0 / 4;
        uint32_t d[4];
        float sv[4], bv[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            d[j] = w[64 * j + lane];
            const size_t e = e0 + 256 * j + 4 * lane;
            const size_t g = gshift >= 0 ? e >> gshift : e / group;
            sv[j] = scales[g];
            bv[j] = biases ? biases[g] : 0.0f;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) st4(out + e0 + 256 * j + 4 * lane, affine4<FMA>(d[j], sv[j], bv[j]));
    });
    for (size_t i = n_full + thread_id(); i < n; i += n_threads()) {
        const size_t g = i / group;
        out[i] = affine<FMA>((float)byte_at(in, i), scales[g], biases ? biases[g] : 0.0f);
    }
}

__device__ __forceinline__ float4 i8x4_to_f32x4_scaled(uint32_t w, float s) {
    return make_float4((float)(int8_t)(w & 0xFFu) * s, (float)(int8_t)((w >> 8) & 0xFFu) * s,
                       (float)(int8_t)((w >> 16) & 0xFFu) * s, (float)(int8_t)(w >> 24) * s);
}

// VEC requires 16-byte aligned pointers and k % 16 == 0 (a lane's 4 elements
// then lie in one row), and n < 2^32 (32-bit row division).
template <bool VEC>
__global__ __launch_bounds__(kThreads) void k_rowwise_dequantize(const int8_t *__restrict__ q,
                                                                 const float *__restrict__ scales,
                                                                 float *__restrict__ out, size_t n,
                                                                 size_t k) {
    const size_t n_full = VEC ? n / kStep * kStep : 0;
    wave_steps(n_full, [&](size_t e0, int lane) {
        const uint32_t *w = reinterpret_cast<const uint32_t *>(q) + e0 / 4;
        uint32_t d[4];
        float sv[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            d[j] = w[64 * j + lane];
            sv[j] = scales[(uint32_t)(e0 + 256 * j + 4 * lane) / (uint32_t)k];
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) st4(out + e0 + 256 * j + 4 * lane, i8x4_to_f32x4_scaled(d[j], sv[j]));
    });
    for (size_t i = n_full + thread_id(); i < n; i += n_threads()) out[i] = (float)q[i] * scales[i / k];
}

unsigned blocks_for(size_t n) {
    size_t chunks = (n + 15) / 16;  // 16 elements per thread
    size_t b = (chunks + kThreads - 1) / kThreads;
    if (b < 1) b = 1;
    if (b > kMaxBlocks) b = kMaxBlocks;
    return (unsigned)b;
}

}  // namespace

int launch_dequantize(const uint32_t *in, size_t n_words, float *out, size_t n_out, hipStream_t s) {
    size_t n = n_words * 4;
    if (n > n_out) n = n_out;
    if (n == 0) return RQ_OK;
    const bool vec = aligned(in, 16) && aligned(out, 16);
    if (vec)
        hipLaunchKernelGGL(k_dequantize<true>, dim3(blocks_for(n)), dim3(kThreads), 0, s, in, out, n);
    else
        hipLaunchKernelGGL(k_dequantize<false>, dim3(blocks_for(n)), dim3(kThreads), 0, s, in, out, n);
    RQ_LAUNCH_CHECK();
    return RQ_OK;
}

int launch_affine_dequantize(const uint32_t *w, const float *scales, const float *biases, float *out,
                             size_t n, uint32_t group, bool fma, hipStream_t s) {
    if (n == 0) return RQ_OK;
    const bool vec = aligned(w, 16) && aligned(out, 16) && group % 16 == 0;
    const int gshift = (group & (group - 1)) == 0 ? __builtin_ctz(group) : -1;
    const dim3 grid(blocks_for(n)), block(kThreads);
    if (vec && fma)
        hipLaunchKernelGGL((k_affine_dequantize<true, true>), grid, block, 0, s, w, scales, biases, out, n, group,
                           gshift);
    else if (vec)
        hipLaunchKernelGGL((k_affine_dequantize<true, false>), grid, block, 0, s, w, scales, biases, out, n, group,
                           gshift);
    else if (fma)
        hipLaunchKernelGGL((k_affine_dequantize<false, true>), grid, block, 0, s, w, scales, biases, out, n, group,
                           gshift);
    else
        hipLaunchKernelGGL((k_affine_dequantize<false, false>), grid, block, 0, s, w, scales, biases, out, n, group,
                           gshift);
    RQ_LAUNCH_CHECK();
    return RQ_OK;
}

int launch_rowwise_dequantize(const int8_t *q, const float *scales, float *out, int64_t n_rows, int64_t k,
                              hipStream_t s) {
    const size_t n = (size_t)n_rows * (size_t)k;
    if (n == 0) return RQ_OK;
    const bool vec = aligned(q, 16) && aligned(out, 16) && k % 16 == 0 && n < ((size_t)1 << 32);
    if (vec)
        hipLaunchKernelGGL(k_rowwise_dequantize<true>, dim3(blocks_for(n)), dim3(kThreads), 0, s, q, scales, out, n,
                           (size_t)k);
    else
        hipLaunchKernelGGL(k_rowwise_dequantize<false>, dim3(blocks_for(n)), dim3(kThreads), 0, s, q, scales, out, n,
                           (size_t)k);
    RQ_LAUNCH_CHECK();
    return RQ_OK;
}

}  // namespace rq
