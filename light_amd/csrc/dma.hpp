// dma.hpp -- direct global -> LDS loads (gfx950 global_load_lds_dword[x4]) and explicit
// vector-memory wait counts.
//
// The loads are issued from inline asm so that the compiler does not treat them as
// pending LDS writes: it would otherwise wait for every outstanding LDS DMA before any LDS
// access, which serialises a multi-stage pipeline.  Callers therefore wait for them
// explicitly with wait_vm<N>() / wait_vm_rt(n): vmcnt counts loads in issue order, so
// "at most N newer loads outstanding" means every older load has landed in LDS.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hq {

// 16 bytes from global memory to LDS at lds_base + lane * 16 (lds_base wave-uniform).
__device__ __forceinline__ void dma16(const void *g, uint32_t lds_base) {
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds_base) : "memory", "m0");
#pragma clang diagnostic pop
}
// 4 bytes from global memory to LDS at lds_base + lane * 4.
__device__ __forceinline__ void dma4(const void *g, uint32_t lds_base) {
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off" ::"v"(g), "s"(lds_base) : "memory", "m0");
#pragma clang diagnostic pop
}

template <int N>
__device__ __forceinline__ void wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Wave-uniform runtime count (0..31).
__device__ __forceinline__ void wait_vm_rt(int n) {
  switch (n) {
#define HQ_WCASE(k) \
  case k:           \
    wait_vm<k>();   \
    break;
    HQ_WCASE(0) HQ_WCASE(1) HQ_WCASE(2) HQ_WCASE(3) HQ_WCASE(4) HQ_WCASE(5) HQ_WCASE(6) HQ_WCASE(7)
    HQ_WCASE(8) HQ_WCASE(9) HQ_WCASE(10) HQ_WCASE(11) HQ_WCASE(12) HQ_WCASE(13) HQ_WCASE(14) HQ_WCASE(15)
    HQ_WCASE(16) HQ_WCASE(17) HQ_WCASE(18) HQ_WCASE(19) HQ_WCASE(20) HQ_WCASE(21) HQ_WCASE(22) HQ_WCASE(23)
    HQ_WCASE(24) HQ_WCASE(25) HQ_WCASE(26) HQ_WCASE(27) HQ_WCASE(28) HQ_WCASE(29) HQ_WCASE(30) HQ_WCASE(31)
#undef HQ_WCASE
    default:
      wait_vm<0>();
  }
}

}  // namespace hq
