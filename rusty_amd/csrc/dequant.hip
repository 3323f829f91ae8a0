// Standalone dequantization kernels for gfx950.
//
//   k_dequantize         <- rusty-backend/src/kernels.wgsl:153-166 (`dequantize`)
//   k_affine_dequantize  <- rusty-backend/src/kernels.wgsl:379-400 (`affine_dequantize`)
//   k_rowwise_dequantize    per-row signed int8: f32(q) * scale[row]
//
// All three are HBM-bound byte expansions (1 B in, 4 B out per element, plus
// the group scalars).  One thread owns a 16-byte chunk of codes: one
// dwordx4 load, four float4 stores, so a wave moves 1 KiB of codes and 4 KiB
// of f32 per step with fully coalesced accesses.  The WGSL runs one
// invocation per element and re-reads the containing u32 four times.
// Chunks that cross the end of the data (or unaligned pointers) take a
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

template <bool VEC>
__global__ __launch_bounds__(kThreads) void k_dequantize(const uint32_t *__restrict__ in,
                                                         float *__restrict__ out, size_t n) {
    const size_t n_chunks = (n + 15) / 16;
    for (size_t c = (size_t)blockIdx.x * kThreads + threadIdx.x; c < n_chunks;
         c += (size_t)gridDim.x * kThreads) {
        const size_t base = c * 16;
        if (VEC && base + 16 <= n) {
            const uint4 w = reinterpret_cast<const uint4 *>(in)[c];
            float4 *o = reinterpret_cast<float4 *>(out + base);
            o[0] = bytes_to_f32x4(w.x);
            o[1] = bytes_to_f32x4(w.y);
            o[2] = bytes_to_f32x4(w.z);
            o[3] = bytes_to_f32x4(w.w);
        } else {
            const size_t end = base + 16 < n ? base + 16 : n;
            for (size_t i = base; i < end; ++i) out[i] = (float)byte_at(in, i);
        }
    }
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

// VEC requires 16-byte aligned pointers and group % 16 == 0 (a chunk then
// lies inside one group).
template <bool VEC, bool FMA>
__global__ __launch_bounds__(kThreads) void k_affine_dequantize(const uint32_t *__restrict__ in,
                                                                const float *__restrict__ scales,
                                                                const float *__restrict__ biases,
                                                                float *__restrict__ out, size_t n,
                                                                uint32_t group) {
    const size_t n_chunks = (n + 15) / 16;
    for (size_t c = (size_t)blockIdx.x * kThreads + threadIdx.x; c < n_chunks;
         c += (size_t)gridDim.x * kThreads) {
        const size_t base = c * 16;
        if (VEC && base + 16 <= n) {
            const size_t g = base / group;
            const float s = scales[g];
            const float b = biases ? biases[g] : 0.0f;
            const uint4 w = reinterpret_cast<const uint4 *>(in)[c];
            float4 *o = reinterpret_cast<float4 *>(out + base);
            o[0] = affine4<FMA>(w.x, s, b);
            o[1] = affine4<FMA>(w.y, s, b);
            o[2] = affine4<FMA>(w.z, s, b);
            o[3] = affine4<FMA>(w.w, s, b);
        } else {
            const size_t end = base + 16 < n ? base + 16 : n;
            for (size_t i = base; i < end; ++i) {
                const size_t g = i / group;
                out[i] = affine<FMA>((float)byte_at(in, i), scales[g], biases ? biases[g] : 0.0f);
            }
        }
    }
}

__device__ __forceinline__ float4 i8x4_to_f32x4_scaled(uint32_t w, float s) {
    return make_float4((float)(int8_t)(w & 0xFFu) * s, (float)(int8_t)((w >> 8) & 0xFFu) * s,
                       (float)(int8_t)((w >> 16) & 0xFFu) * s, (float)(int8_t)(w >> 24) * s);
}

// VEC requires 16-byte aligned pointers and k % 16 == 0 (a chunk then lies in one row).
template <bool VEC>
__global__ __launch_bounds__(kThreads) void k_rowwise_dequantize(const int8_t *__restrict__ q,
                                                                 const float *__restrict__ scales,
                                                                 float *__restrict__ out, size_t n,
                                                                 size_t k) {
    const size_t n_chunks = (n + 15) / 16;
    for (size_t c = (size_t)blockIdx.x * kThreads + threadIdx.x; c < n_chunks;
         c += (size_t)gridDim.x * kThreads) {
        const size_t base = c * 16;
        if (VEC && base + 16 <= n) {
            const float s = scales[base / k];
            const uint4 w = reinterpret_cast<const uint4 *>(q)[c];
            float4 *o = reinterpret_cast<float4 *>(out + base);
            o[0] = i8x4_to_f32x4_scaled(w.x, s);
            o[1] = i8x4_to_f32x4_scaled(w.y, s);
            o[2] = i8x4_to_f32x4_scaled(w.z, s);
            o[3] = i8x4_to_f32x4_scaled(w.w, s);
        } else {
            const size_t end = base + 16 < n ? base + 16 : n;
            for (size_t i = base; i < end; ++i) out[i] = (float)q[i] * scales[i / k];
        }
    }
}

unsigned blocks_for(size_t n) {
    size_t chunks = (n + 15) / 16;
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
    const dim3 grid(blocks_for(n)), block(kThreads);
    if (vec && fma)
        hipLaunchKernelGGL((k_affine_dequantize<true, true>), grid, block, 0, s, w, scales, biases, out, n, group);
    else if (vec)
        hipLaunchKernelGGL((k_affine_dequantize<true, false>), grid, block, 0, s, w, scales, biases, out, n, group);
    else if (fma)
        hipLaunchKernelGGL((k_affine_dequantize<false, true>), grid, block, 0, s, w, scales, biases, out, n, group);
    else
        hipLaunchKernelGGL((k_affine_dequantize<false, false>), grid, block, 0, s, w, scales, biases, out, n, group);
    RQ_LAUNCH_CHECK();
    return RQ_OK;
}

int launch_rowwise_dequantize(const int8_t *q, const float *scales, float *out, int64_t n_rows, int64_t k,
                              hipStream_t s) {
    const size_t n = (size_t)n_rows * (size_t)k;
    if (n == 0) return RQ_OK;
    const bool vec = aligned(q, 16) && aligned(out, 16) && k % 16 == 0;
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
