// Direct global->LDS loads (gfx950 global_load_lds_dwordx4) and the barrier
// that publishes what they brought, shared by the MFMA GEMMs that stage both
// operands this way (kquant_gemm.hip, int8_gemm.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace syn {

// One direct global->LDS load of 16 bytes per lane into lds_addr + 16 * lane
// (lds_addr wave-uniform).  Issued as inline assembly so that the compiler's
// memory-counter bookkeeping does not see it: it would otherwise wait for
// every direct load before the next LDS read it cannot prove disjoint from
// it.  kr_publish waits for these loads explicitly.  M0 (the LDS address)
// is a reserved register: the statement restores its value.
__device__ __forceinline__ void kr_dma(const void *src, uint32_t lds_addr) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %1, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(src), "s"(lds_addr)
      : "memory");
}

// Wait until this wave's direct loads of the next stage have landed (the
// AFTER loads issued since are the stage after next) and its LDS reads of
// the current stage have returned, then meet the other waves, after which
// the current stage may be overwritten.  A plain s_barrier:
// __syncthreads()'s fence would wait for every outstanding load, the
// prefetches included.
template <int AFTER>
__device__ __forceinline__ void kr_publish() {
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(AFTER) : "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// the LDS address of a dynamic shared-memory pointer (the M0 operand above)
template <class T>
__device__ __forceinline__ uint32_t lds_addr_of(T *p) {
  return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) T *)p;
}

}  // namespace syn
