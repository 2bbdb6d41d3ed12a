// Buffer->LDS DMA helpers shared by the prefill kernels (head_dim 64/128 and 256).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace kvq {

// Buffer->LDS DMA issued from inline asm: the compiler does not model these loads, so it adds no
// wait for them before the kernel's LDS accesses; the tile ring orders every slot with explicit
// vmcnt waits and barriers. M0 (the LDS base of the wave's 64 lanes) is saved and restored around
// the load. Lane i's 16 bytes (2 bytes, in the low half of a 4-byte cell) land at lds + 16 i
// (lds + 4 i). `lds` and `so` are wave-uniform; readfirstlane states it to the compiler.
__device__ __forceinline__ void dma_b128(__amdgpu_buffer_rsrc_t r, uint32_t lds, uint32_t vo, uint32_t so) {
  uint32_t m0;
  asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\tbuffer_load_dwordx4 %2, %3, %4 offen lds\n\ts_mov_b32 m0, %0"
               : "=&s"(m0)
               : "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(vo), "s"(r), "s"(__builtin_amdgcn_readfirstlane(so))
               : "memory");
}
__device__ __forceinline__ void dma_b32(__amdgpu_buffer_rsrc_t r, uint32_t lds, uint32_t vo, uint32_t so) {
  uint32_t m0;
  asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\tbuffer_load_dword %2, %3, %4 offen lds\n\ts_mov_b32 m0, %0"
               : "=&s"(m0)
               : "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(vo), "s"(r), "s"(__builtin_amdgcn_readfirstlane(so))
               : "memory");
}
__device__ __forceinline__ void dma_b16(__amdgpu_buffer_rsrc_t r, uint32_t lds, uint32_t vo, uint32_t so) {
  uint32_t m0;
  asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\tbuffer_load_ushort %2, %3, %4 offen lds\n\ts_mov_b32 m0, %0"
               : "=&s"(m0)
               : "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(vo), "s"(r), "s"(__builtin_amdgcn_readfirstlane(so))
               : "memory");
}
// s_waitcnt vmcnt(N), other counters left alone.
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}
__device__ __forceinline__ uint32_t lds_addr(const void* ptr) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)ptr;
}
// A wave-uniform value the compiler treats as unknown. A buffer chosen by it is addressed as the
// lane's offset plus this scalar, rather than by one precomputed vector address per buffer held in
// registers through the loop (the LDS arrays extend past the 64 KiB immediate-offset range).
__device__ __forceinline__ int opaque(int x) {
  asm("" : "+s"(x));
  return x;
}

}  // namespace kvq
