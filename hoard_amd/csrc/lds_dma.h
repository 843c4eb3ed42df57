// Global-to-LDS copies with global_load_lds_dwordx4, issued from inline
// assembly.
//
// The compiler does not see these copies, so it does not make the wave's
// later LDS reads wait for them; the wave that issued a copy waits for it
// itself (lds_dma_wait, i.e. s_waitcnt vmcnt(0)) and, where other waves read
// the data, a barrier follows.  vmcnt counts the copies in issue order
// together with the wave's other vector-memory operations.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hoard {

typedef __attribute__((address_space(3))) void lds_void;

// One 1 KB chunk (64 lanes x 16 bytes): lane l copies the 16 bytes at its
// own source address g to dst[16 l, 16 l + 16).  g must be 16-byte aligned and
// dst a 16-byte aligned LDS address (a generic pointer into a __shared__
// array).  Lanes switched off by the caller copy nothing.
__device__ __forceinline__ void dma_lanes(uint8_t *dst, const uint8_t *g) {
    const lds_void *lp = (const lds_void *)dst;  // generic -> LDS address space: the 32-bit LDS offset
    const uint32_t lds = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(uintptr_t)lp);
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds), "v"(g)
                 : "memory", "m0");
}

// The 4-byte form: lane l copies the 4 bytes at its own source address g to
// dst[4 l, 4 l + 4); g 4-byte aligned, dst a 4-byte aligned LDS address.
__device__ __forceinline__ void dma_lanes4(uint8_t *dst, const uint8_t *g) {
    const lds_void *lp = (const lds_void *)dst;
    const uint32_t lds = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(uintptr_t)lp);
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, off" ::"s"(lds), "v"(g) : "memory", "m0");
}

// The contiguous form: lane l copies src[16 l, 16 l + 16).
__device__ __forceinline__ void dma_chunk(uint8_t *dst, const uint8_t *src) {
    dma_lanes(dst, src + (threadIdx.x & 63) * 16);
}

// The same copy with the non-temporal (streaming) cache policy, for expert
// weights that are read once per call: the caches keep what is read again
// (router rows, activations, exchange words) rather than the stream.
__device__ __forceinline__ void dma_chunk_nt(uint8_t *dst, const uint8_t *src) {
    const lds_void *lp = (const lds_void *)dst;
    const uint32_t lds = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(uintptr_t)lp);
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off nt" ::"s"(lds),
                 "v"(src + (threadIdx.x & 63) * 16)
                 : "memory", "m0");
}

// Copy nbytes (a multiple of 16) from src to dst with the calling wave alone.
__device__ __forceinline__ void dma_wave_copy(uint8_t *dst, const uint8_t *src, int nbytes) {
    const int lane = threadIdx.x & 63;
    for (int c = 0; c < nbytes; c += 1024) {
        if (c + 16 * lane < nbytes) dma_chunk(dst + c, src + c);
    }
}

// dma_wave_copy with the non-temporal cache policy, for expert weights.
__device__ __forceinline__ void dma_wave_copy_nt(uint8_t *dst, const uint8_t *src, int nbytes) {
    const int lane = threadIdx.x & 63;
    for (int c = 0; c < nbytes; c += 1024) {
        if (c + 16 * lane < nbytes) dma_chunk_nt(dst + c, src + c);
    }
}

// Workgroup barrier after this wave's LDS operations: the data the waves
// exchange goes through LDS, so the vector-memory counters need not drain.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Wait for every vector-memory operation of the wave, LDS copies included;
// the memory clobber keeps the compiler from moving LDS reads above it.
__device__ __forceinline__ void lds_dma_wait() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

}  // namespace hoard
