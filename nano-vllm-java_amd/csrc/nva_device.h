// Device helpers shared by the kernels of libnva.so (included by .hip sources only).
#pragma once

#include <hip/hip_runtime.h>

namespace nva {

// Word 3 of a raw (stride 0) buffer descriptor on gfx9-family parts: 32-bit data format, no
// swizzle; out-of-range offsets read zero.
constexpr int kBufferWord3 = 0x00020000;

// 16 bytes per lane from base + off to LDS (lane l's at lds + 4 l), through a buffer
// descriptor over [base, base + bytes): the base stays in scalar registers, the lane offset is
// 32-bit, and the hardware range-checks the read (reads past `bytes` return zeros).
__device__ __forceinline__ void copy16_to_lds(const float *base, int bytes, uint32_t off,
                                              float *lds) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(base), (short)0, bytes,
                                        kBufferWord3),
      (__attribute__((address_space(3))) void *)lds, 16, off, 0, 0, 0);
}

// Asynchronous HBM -> LDS copies that the compiler does not see as LDS writes.
//
// The compiler waits for every outstanding LDS-DMA copy (vmcnt) before an LDS read it cannot
// prove disjoint from them, and across a loop back edge it cannot: a multi-stage ring copied
// with copy16_to_lds above then drains all its prefetches before each read.  The copies below
// are issued from inline assembly instead, so the kernel alone orders them: wait_copies<N>()
// before reading a stage (its copies have landed once at most N later ones are outstanding),
// wait_lds_reads() before a copy overwrites a stage this wave has read, and lds_barrier()
// between waves.  All three are opaque to the compiler and clobber memory, so no LDS access
// moves across them.  The compiler's own waits on its own memory operations stay correct: a
// copy it does not count only makes a vmcnt it computes wait longer.

// LDS byte address of a __shared__ location (wave-uniform).
__device__ __forceinline__ uint32_t lds_address(const void *p) {
  return __builtin_amdgcn_readfirstlane(
      (uint32_t)(size_t)(const __attribute__((address_space(3))) void *)p);
}

// 16 bytes per lane from base + off into LDS at byte address lds + 16 * lane, through a buffer
// descriptor over [base, base + bytes) (reads past `bytes` return zeros).  base, bytes and lds
// are wave-uniform.
__device__ __forceinline__ void copy16_to_lds_async(const float *base, int bytes, uint32_t off,
                                                    uint32_t lds) {
  typedef int v4i __attribute__((ext_vector_type(4)));
  const uint64_t b = (uint64_t)(size_t)base;
  v4i r;
  r.x = __builtin_amdgcn_readfirstlane((int)(uint32_t)b);
  r.y = __builtin_amdgcn_readfirstlane((int)((uint32_t)(b >> 32) & 0xffffu));
  r.z = __builtin_amdgcn_readfirstlane(bytes);
  r.w = kBufferWord3;
  // M0 holds the LDS address; one wait state between writing M0 and the load that reads it.
  asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(off), "s"(r),
               "{m0}"(lds)
               : "memory");
}

// Wait until at most N of this wave's vector memory operations are outstanding.
template <int N> __device__ __forceinline__ void wait_copies() {
  static_assert(N >= 0 && N < 64, "vmcnt is six bits");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Wait until this wave's LDS reads have returned.
__device__ __forceinline__ void wait_lds_reads() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// Workgroup barrier with no implied wait.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_barrier" ::: "memory"); }

// Id (0-7) of the XCD this wave runs on (hardware register XCC_ID, bits 3:0).
__device__ __forceinline__ int xcd_id() { return __builtin_amdgcn_s_getreg((3 << 11) | 20) & 7; }

// The launch's last workgroup (in dispatch order) stores the id of its XCD at hint[0].
__device__ __forceinline__ void record_last_xcd(int32_t *hint) {
  if (hint && threadIdx.x == 0 && blockIdx.x == gridDim.x - 1 && blockIdx.y == gridDim.y - 1 &&
      blockIdx.z == gridDim.z - 1)
    hint[0] = xcd_id();
}

}  // namespace nva
