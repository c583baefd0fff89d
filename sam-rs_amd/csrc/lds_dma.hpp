// LDS DMA helpers for gfx950: global_load_lds (global memory straight into LDS, no registers) and
// explicit vector-memory waits.
//
// The DMAs are issued through inline asm so that the compiler inserts no waits of its own before later
// LDS reads (it cannot tell which LDS region a DMA writes). Kernels wait for them explicitly with
// wait_vm. A wave's vector-memory operations complete in issue order, so wait_vm<N> is correct when N
// counts operations issued after the awaited one; other vector-memory operations in between only make
// the wait longer. The compiler's own waits for its loads count only its own operations, so a load
// issued before DMAs is waited for together with them: kernels load what the compiler tracks before
// the DMAs that should stay in flight past its use, or wait for it in a compiler-visible s_waitcnt.
// M0 is written by every DMA and read by nothing else in these kernels (gfx950 LDS instructions do
// not use it), hence the clobber of a register the compiler reserves.
#pragma once
#include "common.hpp"

#pragma clang diagnostic ignored "-Winline-asm"

namespace samhip {

// Lane l's 16 bytes at base + off land at LDS byte address lds + 16 l. base is wave-uniform (SGPRs),
// off this lane's byte offset from it, lds wave-uniform.
__device__ __forceinline__ void dma16(const void* base, unsigned off, unsigned lds) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "s"(lds)
               : "memory", "m0");
}

// Raw buffer descriptor for `bytes` bytes at p (wave-uniform): buffer loads past the end read 0, range
// checked per dword. Word 3 selects the 32-bit raw data format.
typedef int i32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ i32x4 buffer_rsrc(const void* p, unsigned bytes) {
  const unsigned long a = (unsigned long)p;
  i32x4 r;
  r[0] = __builtin_amdgcn_readfirstlane((int)(unsigned)a);
  r[1] = __builtin_amdgcn_readfirstlane((int)((a >> 32) & 0xffff));
  r[2] = __builtin_amdgcn_readfirstlane((int)bytes);
  r[3] = 0x00020000;
  return r;
}
// dma16 through a buffer descriptor: lane l's 16 bytes at byte offset off land at lds + 16 l; the
// dwords past the descriptor's range land as 0.
__device__ __forceinline__ void bdma16(i32x4 rsrc, unsigned off, unsigned lds) {
  asm volatile("s_mov_b32 m0, %2\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(off), "s"(rsrc), "s"(lds)
               : "memory", "m0");
}

// bdma16 with a wave-uniform byte offset soff added to every lane's offset (buffer soffset).
__device__ __forceinline__ void bdma16s(i32x4 rsrc, unsigned off, unsigned soff, unsigned lds) {
  asm volatile("s_mov_b32 m0, %3\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds" ::"v"(off), "s"(rsrc), "s"(soff), "s"(lds)
               : "memory", "m0");
}

// LDS byte address of a pointer into dynamic shared memory.
__device__ __forceinline__ unsigned lds_addr(const void* p) {
  return (unsigned)(size_t)(const __attribute__((address_space(3))) char*)(p);
}

// ds_read_b64_tr_b16 (the lane layout of lds_read_tr16) at a byte address of the workgroup's LDS.
__device__ __forceinline__ i16x4 lds_read_tr16_at(unsigned addr) {
  typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(size_t)addr);
}

// Hides v's value from the optimiser, so that constants added to it later stay instruction offsets
// instead of being folded into new per-lane base registers.
__device__ __forceinline__ unsigned opaque(unsigned v) {
  asm volatile("" : "+v"(v));
  return v;
}

// Waits until at most N of this wave's vector-memory operations are outstanding, i.e. everything
// issued before the last N is done.
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

}  // namespace samhip
