// Global -> LDS copies and the waits for them (gfx950), shared by the MoE
// kernels that stream weight records through LDS rings.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

// Global -> LDS copies (gfx950 global_load_lds): lane i's bytes land at the
// wave-uniform LDS address base + i * size.  Issued as inline assembly so that
// the compiler does not drain them at the next barrier; their completion is
// waited for explicitly (s_waitcnt vmcnt) before the LDS is read.
__device__ __forceinline__ unsigned lds_addr(const void *p) {
  return (unsigned)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma_b128(const void *gptr, unsigned base) {
  base = __builtin_amdgcn_readfirstlane(base);
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(gptr), "s"(base) : "memory", "m0");
}
// device-scope (sc1): sees other workgroups' atomics once they are done
__device__ __forceinline__ void dma_b128_dev(const void *gptr, unsigned base) {
  base = __builtin_amdgcn_readfirstlane(base);
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off sc1" ::"v"(gptr), "s"(base) : "memory", "m0");
}
__device__ __forceinline__ void dma_b32(const void *gptr, unsigned base) {
  base = __builtin_amdgcn_readfirstlane(base);
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(gptr), "s"(base) : "memory", "m0");
}
// the same copy from a wave-uniform base plus a per-lane 32-bit byte offset
__device__ __forceinline__ void dma_b128_s(const void *sbase, unsigned voff, unsigned base) {
  base = __builtin_amdgcn_readfirstlane(base);
  // the base is wave-uniform by construction; say so to the compiler
  const unsigned long long sb = (unsigned long long)sbase;
  sbase = (const void *)(((unsigned long long)(unsigned)__builtin_amdgcn_readfirstlane((int)(unsigned)(sb >> 32)) << 32) |
                         (unsigned)__builtin_amdgcn_readfirstlane((int)(unsigned)sb));
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "s"(base)
               : "memory", "m0");
}
#pragma clang diagnostic pop
__device__ __forceinline__ void wait_dma() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// s_waitcnt vmcnt(n) for a wave-uniform n (the immediate is encoded per case;
// gfx950's counter holds 6 bits, so n > 63 waits for everything)
__device__ __forceinline__ void wait_vm(int n) {
  switch (n) {
#define SW_VM(k) \
  case k:        \
    asm volatile("s_waitcnt vmcnt(" #k ")" ::: "memory"); \
    break;
    SW_VM(1) SW_VM(2) SW_VM(3) SW_VM(4) SW_VM(5) SW_VM(6) SW_VM(7) SW_VM(8) SW_VM(9) SW_VM(10) SW_VM(11)
    SW_VM(12) SW_VM(13) SW_VM(14) SW_VM(15) SW_VM(16) SW_VM(17) SW_VM(18) SW_VM(19) SW_VM(20) SW_VM(21)
    SW_VM(22) SW_VM(23) SW_VM(24) SW_VM(25) SW_VM(26) SW_VM(27) SW_VM(28) SW_VM(29) SW_VM(30)
    SW_VM(31) SW_VM(32) SW_VM(33) SW_VM(34) SW_VM(35) SW_VM(36) SW_VM(37) SW_VM(38) SW_VM(39) SW_VM(40)
    SW_VM(41) SW_VM(42) SW_VM(43) SW_VM(44) SW_VM(45) SW_VM(46) SW_VM(47) SW_VM(48) SW_VM(49) SW_VM(50)
    SW_VM(51) SW_VM(52) SW_VM(53) SW_VM(54) SW_VM(55) SW_VM(56) SW_VM(57) SW_VM(58) SW_VM(59) SW_VM(60)
    SW_VM(61) SW_VM(62) SW_VM(63)
#undef SW_VM
    default:
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
}
