// hm_lds_dma.h -- direct global -> LDS loads and the waits around them
// (gfx950), shared by the kernels that stage operands through an LDS ring.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// s_waitcnt with only vmcnt constrained (gfx9 encoding: vmcnt bits 3:0 and
// 15:14, expcnt 6:4, lgkmcnt 11:8).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    constexpr int imm = (N & 15) | (((N >> 4) & 3) << 14) | (7 << 4) | (15 << 8);
    __builtin_amdgcn_s_waitcnt(imm);
}

// Ring barrier.  __syncthreads() would also drain every load still in flight
// (vmcnt(0)), emptying the ring.  Here the caller's s_waitcnt vmcnt(N) has
// already completed this wave's loads of the stage being published; the
// lgkmcnt(0) completes this wave's LDS reads and writes (including those of
// the slot refilled right after the barrier).  The memory clobber keeps the
// compiler from moving memory accesses across it.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// The same barrier, leaving this wave's N most recent LDS operations in
// flight (LDS operations complete in issue order; the caller keeps scalar
// memory loads out of the window so that the count holds LDS operations
// only).
template <int N>
__device__ __forceinline__ void lds_barrier_keep() {
    static_assert(N >= 0 && N <= 15, "lgkmcnt range");
    asm volatile("s_waitcnt lgkmcnt(%0)\n\ts_barrier" ::"n"(N) : "memory");
}

// One wave-wide 16-byte global -> LDS load: lane l's 16 bytes from its own
// gsrc land at lds_base + 16*l (M0 holds the wave-uniform LDS base).
//
// Written as inline asm rather than __builtin_amdgcn_global_load_lds: the
// compiler cannot follow which ring slot an in-flight LDS load targets across
// the K loop's back edge and then drains every load (vmcnt(0)) once per
// iteration.  Here the kernels order the loads themselves: wait_vmcnt before
// reading a stage, lds_barrier before refilling a slot.  The statement sets
// M0 itself, and the kernels hold nothing else in M0 (no LDS DMA through the
// builtin, no indirect register indexing, no GWS or messages).  The memory
// clobber keeps other memory accesses on their side of the load.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(const void* gsrc, void* lds_base) {
    const unsigned m0 = (unsigned)(uintptr_t)(lds_ptr_t)lds_base;
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off"
                 :: "v"(gsrc), "s"(m0) : "memory", "m0");
}
// The same with 4 bytes per lane: lane l's dword lands at lds_base + 4*l.
// Used for per-row metadata gathers (token ids, scales) that ride in the
// same in-order load queue as the operand stages.
__device__ __forceinline__ void dma4(const void* gsrc, void* lds_base) {
    const unsigned m0 = (unsigned)(uintptr_t)(lds_ptr_t)lds_base;
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off"
                 :: "v"(gsrc), "s"(m0) : "memory", "m0");
}
#pragma clang diagnostic pop
