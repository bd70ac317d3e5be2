// LDS DMA (global_load_lds) issued as inline assembly, and the vmcnt wait
// that orders it, shared by the split-operand screen (emh_screen4.h) and the
// queued-row scan (emh_verify.hip).
#pragma once

#include <cstdint>

#include <hip/hip_runtime.h>

namespace emh {
namespace {

// s_waitcnt vmcnt(N) with the other counters left alone (gfx9 encoding:
// vmcnt in bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// LDS DMA: each lane moves 16 (or 4) bytes from its global address to
// lds + 16 lane (4 lane); lds is wave-uniform (M0 holds its LDS address).
// Issued as inline assembly, which the compiler's wait counting does not
// see: the kernel orders these DMAs against its LDS reads itself (vmcnt
// waits and barriers), where the compiler, unable to tell the ring's stages
// apart across loop iterations, would wait for every DMA in flight before
// each read. (Other loads the compiler waits for stay correct: DMAs it does
// not count only make its vmcnt waits stricter.) M0 is saved and restored
// around the DMA, so no value the compiler keeps there is disturbed.
__device__ __forceinline__ uint32_t lds_addr(const void* lds) {
  return __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)lds);
}
// From a wave-uniform base plus a 32-bit per-lane byte offset.
__device__ __forceinline__ void dma16o(const void* base, uint32_t off, void* lds) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\t"
      "global_load_lds_dwordx4 %1, %2\n\ts_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(off), "s"(base), "s"(lds_addr(lds))
      : "memory");
}
__device__ __forceinline__ void dma4(const void* g, void* lds) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\t"
      "global_load_lds_dword %1, off\n\ts_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(g), "s"(lds_addr(lds))
      : "memory");
}

// From a per-lane 64-bit global address.
__device__ __forceinline__ void dma16(const void* g, void* lds) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\t"
      "global_load_lds_dwordx4 %1, off\n\ts_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(g), "s"(lds_addr(lds))
      : "memory");
}

}  // namespace
}  // namespace emh
