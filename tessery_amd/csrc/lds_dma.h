// LDS DMA helpers for gfx950 kernels that stage tiles with global_load_lds_dwordx4, and asm
// register loads whose waits the kernel places itself.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.h"

namespace tessery {

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// Wait states inside these asm statements. The compiler's hazard padding does not look into
// inline asm, and CDNA3/gfx950 require (AMD's CDNA3 ISA guide, "Manually Inserted Wait States"):
// 5 wait states between a VALU write of an SGPR (v_readlane restoring a spilled SGPR,
// v_readfirstlane) and a vector memory instruction that reads that SGPR as its base address, and
// 1 between an SALU write of M0 and an LDS DMA that reads it. Every asm vector memory instruction
// below is therefore preceded, inside its own statement, by at least 5 wait states (s_nop 4, plus
// the s_mov to M0 where there is one), whatever the compiler placed before the statement.
//
// 16 bytes per lane, global -> LDS (global_load_lds_dwordx4): lane l's bytes land at the
// wave-uniform LDS address + 16*l. Issued as inline asm so the compiler's wait insertion does not
// treat the in-flight DMA as aliasing every later LDS read (it would wait for the whole ring);
// completion is awaited explicitly with wait_vmcnt before the consuming barrier.
__device__ __forceinline__ void dma16(const void* src, _Float16* lds) {
  const unsigned addr = __builtin_amdgcn_readfirstlane(
      static_cast<unsigned>(reinterpret_cast<uintptr_t>((lds_ptr_t)(lds))));
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 4\n\tglobal_load_lds_dwordx4 %0, off"
               :
               : "v"(src), "s"(addr)
               : "memory", "m0");
}

// The same DMA addressed as a wave-uniform 64-bit base (SGPR pair) plus a per-lane unsigned 32-bit
// byte offset: the per-lane address arithmetic stays 32-bit.
__device__ __forceinline__ void dma16_at(const void* base, uint32_t off, _Float16* lds) {
  const unsigned addr = __builtin_amdgcn_readfirstlane(
      static_cast<unsigned>(reinterpret_cast<uintptr_t>((lds_ptr_t)(lds))));
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 4\n\tglobal_load_lds_dwordx4 %0, %1"
               :
               : "v"(off), "s"(base), "s"(addr)
               : "memory", "m0");
}

// 16 bytes per lane, global -> VGPRs, at a wave-uniform base (SGPR pair) plus a per-lane 32-bit
// byte offset and an immediate. Inline asm like the LDS DMA, so the compiler places no waits of
// its own for it (it cannot count the DMAs, and its waits for mixed streams degrade to
// vmcnt(0)); the caller reads dst only after wait_vmcnt_pin. dst is a read-write operand: every
// read of its previous value is ordered before the load (or reads a copy made before it).
template <int OFF>
__device__ __forceinline__ void load16_at(floatx4& dst, const void* base, uint32_t off) {
  asm volatile("s_nop 4\n\tglobal_load_dwordx4 %0, %1, %2 offset:%3"
               : "+v"(dst)
               : "v"(off), "s"(base), "i"(OFF)
               : "memory");
}

// 4 bytes per lane, global -> a VGPR, addressed like load16_at.
template <int OFF>
__device__ __forceinline__ void load4_at(float& dst, const void* base, uint32_t off) {
  asm volatile("s_nop 4\n\tglobal_load_dword %0, %1, %2 offset:%3"
               : "+v"(dst)
               : "v"(off), "s"(base), "i"(OFF)
               : "memory");
}

// The register counts as written here: placed after an s_waitcnt (volatile asm keeps its order
// with the wait), it orders every later read of an asm-loaded register after that wait.
template <typename T>
__device__ __forceinline__ void pin_reg(T& x) {
  asm volatile("" : "+v"(x));
}

// s_waitcnt vmcnt(N); the four registers count as written here, so nothing reads them earlier.
template <int N>
__device__ __forceinline__ void wait_vmcnt_pin(floatx4 (&r)[4]) {
  asm volatile("s_waitcnt vmcnt(%4)"
               : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3])
               : "n"(N)
               : "memory");
}

// s_waitcnt vmcnt(N) pinning six registers (see wait_vmcnt_pin).
template <int N>
__device__ __forceinline__ void wait_vmcnt_pin6(floatx4* r) {
  asm volatile("s_waitcnt vmcnt(%6)"
               : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3]), "+v"(r[4]), "+v"(r[5])
               : "n"(N)
               : "memory");
}

// s_waitcnt vmcnt(n), leaving expcnt / lgkmcnt unconstrained (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// s_waitcnt lgkmcnt(n): this wavefront's LDS reads (and scalar loads) down to n in flight.
template <int N>
__device__ __forceinline__ void wait_lgkmcnt() {
  static_assert(N >= 0 && N < 16, "lgkmcnt range");
  __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4) | (N << 8));
}

// Workgroup barrier without a memory fence. Each wavefront has already waited (vmcnt) for its
// own DMA writes into the stage it is about to release, so after s_barrier every wavefront's
// tile data is in LDS; the asm clobbers keep the compiler from moving LDS accesses across.
// (__syncthreads() would add a release fence that waits for ALL outstanding DMA, including the
// tiles still being prefetched.)
__device__ __forceinline__ void stage_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

}  // namespace tessery
