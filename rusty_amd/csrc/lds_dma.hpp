// Buffer resources and global -> LDS DMA for gfx950 (CDNA4), shared by the
// kernels that stage operands through LDS rings (gemm.hip, matmul_f32.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace rq {

typedef __attribute__((address_space(3))) void lds_void;

// A raw buffer over `bytes` bytes: loads past the end read as zero and never
// touch memory (the bound is what keeps every load of a ring in range).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), 0, bytes, 0x00020000);
}

// A resource whose base and size are wave-uniform values the compiler might
// still hold in VGPRs (the DMA's inline asm takes its resource in SGPRs):
// both are passed through readfirstlane first.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc_s(const void *p, uint32_t bytes) {
    const uint64_t a = reinterpret_cast<uint64_t>(p);
    const uint64_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)a);
    const uint64_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32));
    return make_rsrc(reinterpret_cast<const void *>((hi << 32) | lo),
                     (uint32_t)__builtin_amdgcn_readfirstlane((int)bytes));
}

// The 32-bit LDS address of a __shared__ object.
template <typename T>
__device__ __forceinline__ uint32_t lds_addr(T *p) {
    return (uint32_t)(uintptr_t)(lds_void *)p;
}

// DMA of 16 bytes per lane: LDS[lds_addr + 16 * lane] = buffer[voff], with
// lds_addr a 32-bit LDS address (uniform across the wave).  Issued
// as inline asm so the compiler does not turn its conservative LDS-DMA alias
// tracking into a full vmcnt(0) wait before every LDS read; every reader of a
// stage waits with an explicit s_waitcnt vmcnt instead.  M0 carries the LDS
// base (one wait state before the load, as the ISA requires).  The compiler
// reserves M0 and warns that the "m0" clobber is not honoured (-Winline-asm):
// that is safe only while nothing else in these kernels holds a value in M0
// across a DMA, and in the device assembly of gemm.hip and matmul_f32.hip the
// only instructions naming M0 are these moves (each directly before its load).
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, uint32_t lds_addr, uint32_t voff) {
    const uint32_t l = __builtin_amdgcn_readfirstlane(lds_addr);
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                 :
                 : "s"(l), "v"(voff), "s"(r)
                 : "memory", "m0");
}

// DMA of 4 bytes per lane: LDS[lds_addr + 4 * lane] = buffer[voff].
__device__ __forceinline__ void dma4(__amdgpu_buffer_rsrc_t r, uint32_t lds_addr, uint32_t voff) {
    const uint32_t l = __builtin_amdgcn_readfirstlane(lds_addr);
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dword %1, %2, 0 offen lds"
                 :
                 : "s"(l), "v"(voff), "s"(r)
                 : "memory", "m0");
}

// Waits until at most N vector-memory operations of this wave are outstanding
// (they retire in issue order).  Inline asm with a memory clobber, so the
// compiler cannot move LDS reads of the landed data above the wait.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// Waits until every LDS read of this wave has returned its data.
__device__ __forceinline__ void wait_lgkm0() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

}  // namespace rq
