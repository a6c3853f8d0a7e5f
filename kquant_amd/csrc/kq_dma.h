// Direct HBM -> LDS loads for gfx950 (buffer_load_dwordx4 ... lds).
//
// One instruction moves 16 bytes per lane from a buffer resource straight
// into LDS at m0 + 16 * lane, without passing through VGPRs, so a kernel can
// keep several stages of loads in flight and wait for them with partial
// vmcnt waits.  The loads are issued as assembly, so the compiler does not
// track them: a kernel waits itself (s_waitcnt with waitcnt_vm) and then
// crosses a barrier with a compiler memory clobber, so no LDS read is moved
// above the wait.  Offsets at or past the resource's size read as zero
// without touching memory, which is how these kernels fill padding rows.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace kq {
namespace dma {

typedef int i32x4_t __attribute__((ext_vector_type(4)));

// Largest byte range one resource may cover: offsets are 32-bit and a kernel
// adds at most a 4 KiB in-row offset to a row base.
constexpr uint64_t MAX_RANGE = 0xFFFFF000ull;

// Buffer resource over [base, base + nbytes): raw addressing, range-checked
// (out-of-range offsets read as zero); dword 3 is the gfx9 default format.
__device__ __forceinline__ i32x4_t make_rsrc(const void* base, uint32_t nbytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  i32x4_t r;
  r[0] = (int)(uint32_t)a;
  r[1] = (int)(uint32_t)(a >> 32) & 0xffff;
  r[2] = (int)nbytes;
  r[3] = 0x00020000;
  return r;
}

// s_waitcnt immediate (gfx9 encoding) for vmcnt(N), other counters untouched.
constexpr int waitcnt_vm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

// 16 bytes per lane from rsrc + voffset straight into LDS at m0 + 16 * lane.
__device__ __forceinline__ void load_to_lds16(i32x4_t rsrc, uint32_t voffset, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :
               : "s"(lds_addr), "v"(voffset), "s"(rsrc)
               : "memory", "m0");
}

// 4 bytes per lane from rsrc + voffset (4-byte aligned) into LDS at m0 + 4 * lane.
__device__ __forceinline__ void load_to_lds4(i32x4_t rsrc, uint32_t voffset, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, 0 offen lds"
               :
               : "s"(lds_addr), "v"(voffset), "s"(rsrc)
               : "memory", "m0");
}

// LDS byte address of a __shared__ object.
__device__ __forceinline__ uint32_t lds_offset_of(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) unsigned char*)p;
}

// Wait until at most N of this wave's direct loads are outstanding, then
// barrier: after it every wave's older loads have landed in LDS and every
// wave has finished the LDS reads it issued before the barrier.  The barrier
// builtin does not order memory accesses by itself, so compiler memory
// clobbers on both sides keep every LDS access on its side of it.
template <int N>
__device__ __forceinline__ void wait_and_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(waitcnt_vm(N));
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

}  // namespace dma
}  // namespace kq
