// Device helpers for kernels that stream tiles straight into LDS.
#pragma once
#include "vx_common.h"

// One 16-byte-per-lane load from global memory straight into LDS
// (global_load_lds_dwordx4: lane L's 16 bytes land at lds + 16 L; lds must be
// uniform across the wave, `base` uniform, `off` per lane).  Issued from
// inline asm so that the compiler does not track it: its own waits for LDS
// DMA would drain a prefetch in flight before every LDS read.  Callers order
// it with explicit vmcnt waits.  M0 (the LDS base) is saved and restored
// around it, with the one wait state an M0 write needs before the load.
__device__ __forceinline__ void vx_dma16(const void *base, uint32_t off, uint32_t lds) {
    uint32_t saved;
    __asm__ volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %3\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %1, %2\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(off), "s"(base), "s"(lds)
        : "memory");
}

// As vx_dma16 with 4 bytes per lane (global_load_lds_dword): lane L's dword
// lands at lds + 4 L.
__device__ __forceinline__ void vx_dma4(const void *base, uint32_t off, uint32_t lds) {
    uint32_t saved;
    __asm__ volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %3\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dword %1, %2\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(off), "s"(base), "s"(lds)
        : "memory");
}

// LDS byte address of a __shared__ object.
__device__ __forceinline__ uint32_t vx_lds_addr(const void *p) {
    return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void *)p;
}

// Workgroup barrier for LDS hand-offs only: waits for this wave's LDS
// operations, not for its outstanding global loads (__syncthreads would also
// drain a direct-to-LDS prefetch in flight).
__device__ __forceinline__ void vx_lds_barrier() {
    __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    __asm__ volatile("" ::: "memory");
}

// A pointer the compiler treats as wave-uniform (scalar loads through it).
template <typename T>
__device__ __forceinline__ const T *vx_uniform_ptr(const T *p) {
    const uint64_t v = (uint64_t)(uintptr_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return (const T *)(uintptr_t)(((uint64_t)hi << 32) | lo);
}
