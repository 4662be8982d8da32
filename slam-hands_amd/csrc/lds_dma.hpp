// Direct-to-LDS loads and the explicit waits and barriers that order them
// (gfx950), shared by the kernels that stage operands this way.
#pragma once

#include <hip/hip_runtime.h>

namespace slk {

// One direct-to-LDS load per lane (16 or 4 bytes): lane l reads p and writes
// LDS bytes m0 + size*l (m0 = the wave's region). As inline assembly the
// compiler does not track these LDS writes, so it inserts no waits for them
// before the LDS accesses it cannot prove disjoint (which, in the tile loop,
// would mean waiting for every chunk in flight). Every read of staged data is
// ordered by the explicit vmcnt waits and barriers of the chunk loop.
__device__ __forceinline__ void dma_x4(const void* p, unsigned lds) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(p), "{m0}"(lds) : "memory");
}
__device__ __forceinline__ void dma_x1(const void* p, unsigned lds) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(p), "{m0}"(lds) : "memory");
}
__device__ __forceinline__ unsigned lds_addr(const void* p) { return (unsigned)(size_t)p; }

// s_waitcnt immediates (gfx9 encoding: vmcnt bits 3:0 and 15:14, expcnt 6:4,
// lgkmcnt 11:8): vmcnt(n) lgkmcnt(0) is 0x0070 | n for n < 16; vmcnt(0)
// lgkmcnt(0), and lgkmcnt(0) alone
constexpr int kWaitVm0Lgkm0 = 0x0070;
constexpr int kWaitLgkm0 = 0xC07F;

// Workgroup barrier for LDS hand-offs only: this wave's LDS accesses are
// complete, but its global stores may still be in flight (__syncthreads'
// fence would wait for those too).
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

}  // namespace slk
