// Direct-to-LDS buffer loads (gfx950 `buffer_load_* ... lds`): the loaded
// data goes straight to LDS, not through registers, so a workgroup can keep
// many stages of operands in flight at no register cost.  The LDS address
// is M0 (+ the instruction offset): lane l's data lands at M0 + size*l.
// They are issued from inline assembly so that the compiler inserts no wait
// of its own after them; kernels wait with wait_vmcnt<N>() (loads retire in
// issue order, and the LDS write is done when the count drops).
#pragma once

#include "nhip_internal.h"

namespace nhip {
namespace dma {

// Raw buffer resource over [base, base + bytes): offsets at or past `bytes`
// read as zero without touching memory.  Only the per-lane offset `voff` is
// range checked: an offset that may fall outside goes there, and `soff`
// carries only offsets known to stay inside.
__device__ __forceinline__ v4i raw_rsrc(const void* base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  // word 3 = 0x00020000: the gfx9-family (incl. gfx950) raw-buffer format
  return v4i{(int)(uint32_t)a, (int)(uint32_t)(a >> 32) & 0xffff, (int)bytes, 0x00020000};
}

// 1 KB per wave: lane l's 16 bytes from the buffer at voff + soff to LDS
// byte address lds_base + 16*l.
__device__ __forceinline__ void copy16(uint32_t lds_base, uint32_t voff, v4i rsrc, uint32_t soff) {
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %1, %2, %3 offen lds" ::"s"(lds_base),
      "v"(voff), "s"(rsrc), "s"(soff)
      : "memory", "m0");
}

// 256 bytes per wave: lane l's 4 bytes from the buffer at voff + soff to LDS
// byte address lds_base + 4*l.
__device__ __forceinline__ void copy4(uint32_t lds_base, uint32_t voff, v4i rsrc, uint32_t soff) {
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0\n\t"
      "buffer_load_dword %1, %2, %3 offen lds" ::"s"(lds_base),
      "v"(voff), "s"(rsrc), "s"(soff)
      : "memory", "m0");
}

// Wait until at most N of this wave's vector memory loads are outstanding
// (gfx9 encoding: vmcnt in bits 3:0 and 15:14, expcnt and lgkmcnt left at
// their maximum, i.e. not waited for).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is a 6-bit count");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

}  // namespace dma
}  // namespace nhip
