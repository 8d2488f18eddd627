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

}  // namespace nva
