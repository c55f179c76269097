// cbq_lds_dma.h - gfx950 LDS-DMA primitives shared by the MFMA GEMM kernels:
// global_load_lds_dwordx4 with an explicit M0, the matching wait + barrier,
// and wave-uniform pointers for the DMA's scalar base operand.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cbq {

// LDS DMA of 16 bytes per lane: global sbase + voff -> LDS byte address lds +
// 16 * lane (lds is wave-uniform). M0 carries the LDS address; it is saved
// and restored inside the statement. An LDS DMA needs one wait state after
// the write of M0 it reads (the s_nop; the compiler adds the same one to
// its own M0 writes before such a load).
__device__ __forceinline__ void lds_dma16(uint32_t voff, const void* sbase, uint32_t lds) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %3\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, %2\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(voff), "s"(sbase), "s"(lds)
      : "memory");
}

// Wait until at most N vector-memory operations (the LDS DMAs of later tiles)
// are outstanding and all LDS reads have returned, then barrier. Written as
// one asm statement so that no LDS access is moved across it.
template <int N>
__device__ __forceinline__ void dma_wait_barrier() {
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

// A wave-uniform pointer in SGPRs (the DMA's scalar base operand).
template <typename T>
__device__ __forceinline__ const T* uniform_ptr(const T* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32));
  return reinterpret_cast<const T*>((static_cast<uint64_t>(hi) << 32) | lo);
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p));
}

}  // namespace cbq
