// Global -> LDS loads (global_load_lds_dword / _dwordx4) and explicit vmcnt
// waits, shared by the kernels that stream operand tiles into LDS without
// passing them through registers.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace mb {

typedef __attribute__((address_space(3))) void lds_void_t;

// s_waitcnt with vmcnt = n (n < 16), expcnt and lgkmcnt left at their maxima
// (gfx9 encoding)
#define MB_WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt(0x0F70 | (n))
// The same for any constant n in 0 .. 63 (vmcnt bits [3:0] and [15:14]).
#define MB_WAIT_VMCNT64(n) \
  __builtin_amdgcn_s_waitcnt(((n) & 15) | (((n) >> 4) << 14) | 0x0F70)

// global -> LDS loads (global_load_lds_dword / _dwordx4): lane L's bytes land
// at LDS byte address lds + size * L.  Issued as inline assembly so the
// compiler does not treat them as LDS writes: it would otherwise wait for
// every outstanding load (the two tiles in flight) before each LDS read of
// the tile being computed.  The kernel waits for them itself (MB_WAIT_VMCNT
// before the barrier that publishes a tile).  Loads the compiler cannot see
// only make its own vmcnt waits stricter, never looser.  m0 carries the LDS
// base; the statement saves and restores it, so no register the compiler
// owns changes under it.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(lds_void_t*)p;
}
// Each lane reads base + off (base and `lds` wave-uniform, held in SGPRs;
// off a per-lane byte offset), the scalar-base form of the global load, so a
// tile's addresses cost no vector instructions: the per-lane offsets are
// fixed and the base advances with the tile.
__device__ __forceinline__ uint64_t sgpr_ptr(const void* p) {
  const uint64_t v = (uint64_t)(uintptr_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ void dma16(const void* base, uint32_t off, uint32_t lds) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\t"
      "global_load_lds_dwordx4 %1, %2\n\ts_mov_b32 m0, %0"
      : "=&s"(saved) : "v"(off), "s"(sgpr_ptr(base)), "s"(__builtin_amdgcn_readfirstlane(lds))
      : "memory");
}
__device__ __forceinline__ void dma4(const void* base, uint32_t off, uint32_t lds) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\t"
      "global_load_lds_dword %1, %2\n\ts_mov_b32 m0, %0"
      : "=&s"(saved) : "v"(off), "s"(sgpr_ptr(base)), "s"(__builtin_amdgcn_readfirstlane(lds))
      : "memory");
}


}  // namespace mb
