// Direct global-to-LDS loads (global_load_lds_dword[x4]) and the waits that
// go with them, shared by the kernels that stage tiles in LDS.
//
// The loads go through inline assembly: the compiler's own builtin makes it
// wait for every outstanding load (vmcnt(0)) before any LDS read, which
// would serialise a multi-stage ring. M0 holds the LDS base of the load;
// nothing else in these kernels uses M0.
#pragma once
#include <cstdint>

namespace wg {

// 16 bytes a lane from `src` into LDS at byte address lds + 16 * lane (lds
// uniform across the wave); lanes switched off by a branch load nothing.
__device__ inline void dma16(const void *src, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds), "v"(src)
               : "memory");
}
// The same from base + off: a wave-uniform 64-bit base in SGPRs (stepped by
// scalar adds) and a 32-bit per-lane byte offset, so a stream that advances
// by a fixed stride costs no vector instructions a step.
__device__ inline void dma16(const void *base, uint32_t off, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds), "v"(off),
               "s"(base)
               : "memory");
}
__device__ inline void dma4(const void *base, uint32_t off, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, %2" ::"s"(lds), "v"(off),
               "s"(base)
               : "memory");
}
// 4 bytes a lane into LDS at lds + 4 * lane.
__device__ inline void dma4(const void *src, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, off" ::"s"(lds), "v"(src)
               : "memory");
}

// s_waitcnt vmcnt(N) (gfx9 encoding: vmcnt in bits 3:0 and 15:14). A
// direct-to-LDS load counts as done once its bytes are in LDS.
template <int N>
__device__ inline void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}

// A workgroup barrier that is also a compiler memory barrier but, unlike
// __syncthreads, leaves the hardware counters alone (no vmcnt(0)).
__device__ inline void barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

}  // namespace wg
