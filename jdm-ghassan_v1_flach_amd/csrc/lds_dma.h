// Direct global -> LDS transfers (global_load_lds_dwordx4) issued from inline
// assembly, for kernels that stream operands into LDS without a register
// round trip. Each lane moves 16 bytes to lds_base + 16 * lane (M0 holds the
// wave-uniform LDS base). The compiler does not know these transfers: the
// kernels wait for them with explicit s_waitcnt vmcnt(n), counting their own
// transfers in issue order (the counter is in-order), and synchronise with
// lds_barrier(), which unlike __syncthreads does not drain them.
// M0 is a register the compiler reserves (it rejects a clobber on it): the code relies on no
// compiler-generated instruction using M0 in the kernels that call these, which
// tests/test_abi_cpu.py checks on the generated code of every such file.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gh {

// 64-bit address per lane
__device__ __forceinline__ void lds_dma16(const void* gptr, uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(gptr), "s"(lds_base) : "memory");
}
// 64-bit base in SGPRs + 32-bit per-lane offset (no per-lane address arithmetic)
__device__ __forceinline__ void lds_dma16s(const void* base, uint32_t voff, uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(base), "s"(lds_base) : "memory");
}
// wave-uniform LDS byte address of p
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)p);
}
// block barrier that waits for this wave's LDS operations only
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
__device__ __forceinline__ void lds_wait_lgkm() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }
// wait until at most `ahead` groups of N transfers are outstanding (vmcnt takes an immediate)
template <int N>
__device__ __forceinline__ void lds_dma_wait(int ahead) {
    if (ahead >= 3) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(3 * N) : "memory");
    else if (ahead == 2) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * N) : "memory");
    else if (ahead == 1) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

}  // namespace gh
