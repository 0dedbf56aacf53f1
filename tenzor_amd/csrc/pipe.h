// Pipeline primitives shared by the kernels that stream operand tiles into
// LDS with the gfx950 direct-to-LDS loads (gemm_pipe.hip, mlp.hip): the load
// itself, the LDS-only workgroup barrier, explicit vmcnt waits, and the
// tanh-form GELU of the bias epilogues.  The CPU emulation
// (tests/cpu_emu/hip/hip_runtime.h) supplies its own dma16,
// lds_barrier_only, vmem_*_issued and wave_lds_order.
#pragma once

#include "common.h"

#ifndef TZH_EMULATION
// global_load_lds_dwordx4: lane l's 16 bytes at sbase + voff[l] land in LDS
// at lds_base + 16*l.  Written as asm so that the compiler does not treat
// the ring's loads as pending LDS writes (it would wait for all of them
// before every LDS read); completion is tracked with explicit vmcnt waits.
// M0 is set here and used by nothing else in these kernels.
__device__ __forceinline__ void dma16(const char *sbase, uint32_t voff, char *lds_base) {
    const uint32_t m0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char *)lds_base;
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(m0), "v"(voff), "s"(sbase)
                 : "memory", "m0");
}

// Workgroup barrier for LDS traffic.  The caller has waited for its own LDS
// ops (lgkmcnt); the memory clobber keeps the compiler from moving LDS
// accesses across it, and no fence means no wait for the ring's loads.
__device__ __forceinline__ void lds_barrier_only() { asm volatile("s_barrier" ::: "memory"); }

// Mark a vector store / load the stage waits count (the CPU emulation keeps
// its own in-order record of vector memory ops; on the GPU vmcnt does).
__device__ __forceinline__ void vmem_store_issued() {}
__device__ __forceinline__ void vmem_load_issued() {}

// Orders a wave's LDS writes before its later LDS reads of what other lanes
// of the same wave wrote.  The LDS performs one wave's operations in issue
// order, so only the compiler has to be kept from reordering them.
__device__ __forceinline__ void wave_lds_order() { asm volatile("" ::: "memory"); }
#endif

// Scheduling fence: the compiler moves no instruction across it, so the
// fragment reads and ring loads issued before it go out before the matrix
// products after it (left to itself, it issues each group's reads right
// before the products that consume them, exposing the LDS latency).
__device__ __forceinline__ void sched_fence() {
#ifndef TZH_EMULATION
    __builtin_amdgcn_sched_barrier(0);
#endif
}

// This lane's index in its wave, formed from nothing (v_mbcnt over a full
// mask) and opaque to the compiler: values derived from it are recomputed
// where they are used instead of being held in registers through a kernel.
__device__ __forceinline__ int lane_now() {
#ifdef TZH_EMULATION
    return emu::lane_id();
#else
    int l = __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
    asm volatile("" : "+v"(l));
    return l;
#endif
}

// s_waitcnt vmcnt(N) lgkmcnt(0) (gfx9 encoding; expcnt left at its maximum).
template <int N>
__device__ __forceinline__ void wait_vm_lgkm0() {
    static_assert(N >= 0 && N <= 63, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4));
}

__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt, expcnt not waited for
    lds_barrier_only();
}

__device__ __forceinline__ float gelu_fast(float x) {
    // tanh-form GELU (arctic.zig:750-756): 0.5 x (1 + tanh(u)) = x / (1 + exp(-2u))
    // with u = sqrt(2/pi) (x + 0.044715 x^3); exp and 1/d by v_exp_f32 and
    // v_rcp_f32, about 1 ulp each.
    // x -> -inf: exp -> +inf, 1/d -> 0, result -0; x -> +inf: result x.
    constexpr float c0 = -2.0f * 0.7978845608f * 1.4426950408889634f;  // -2 sqrt(2/pi) log2(e)
    constexpr float c1 = c0 * 0.044715f;
    const float e = __builtin_amdgcn_exp2f(x * __builtin_fmaf(x * x, c1, c0));
    return x * __builtin_amdgcn_rcpf(e + 1.0f);
}
