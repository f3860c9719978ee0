// Direct global -> LDS copies (gfx950 global_load_lds_dwordx4), shared by the kernels that stage
// their operands in LDS rings (K6, K4a).
#pragma once

#include "common.h"

namespace mdl {

// LDS byte address of a pointer into __shared__ memory
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return static_cast<uint32_t>(
      reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) void*)(p)));
}

// s_waitcnt immediate (gfx9 encoding: vmcnt bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8) for
// vmcnt(0) lgkmcnt(0).  Issued through __builtin_amdgcn_s_waitcnt, the wait is visible to the
// compiler's own wait insertion, which then counts every load it issued before as complete.
constexpr int kWaitAll = 0x0070;

// 16 bytes per lane from global memory straight into LDS: lane l's bytes land at lds + 16 l
// (lds wave-uniform, through M0).  Issued as inline assembly, so the compiler neither sees nor
// waits for these loads: a kernel waits for them itself (s_waitcnt vmcnt) before the barrier
// that publishes the stage.  The compiler's own waits stay correct beside them: vector memory
// operations complete in issue order, so loads it does not know of only make its vmcnt(n) waits
// stricter.  Stricter is slower, though: a compiler wait for one of its own loads issued before
// a copy also waits for the copy, so a kernel keeps its own loads and stores out of the way of
// the copies in flight (batched ahead of them, or retired by a builtin wait the compiler sees).
// Kernels that use this must not spill: the library build rejects scratch use in the files that
// include this header.
//
// M0 is written here without the compiler knowing (it does not honour M0 in a clobber list, a
// reserved register).  That is safe only while the compiler itself keeps nothing in M0 in these
// kernels, so the library build also reads their device assembly and fails if any instruction
// outside these asm blocks names M0 (mdlarc_scale_amd/build.py, check_m0).  The compiler's own
// builtin for this copy (__builtin_amdgcn_global_load_lds) sets M0 itself, but its wait
// insertion then puts an s_waitcnt vmcnt(0) before the LDS reads of the current stage, which also
// waits for the copies of the stages ahead: the prefill projections ran 5-7% slower with it.
__device__ __forceinline__ void dma16(const void* src, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
               :: "v"(src), "s"(lds) : "memory");
}

// dma16 from base + off: a wave-uniform (scalar) base address and a per-lane byte offset, so a
// kernel that walks a buffer moves one scalar pointer instead of recomputing lane addresses.
__device__ __forceinline__ void dma16_sbase(const void* base, uint32_t off, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :: "v"(off), "s"(base), "s"(lds) : "memory");
}

}  // namespace mdl
