// Device helpers shared by the kernels: raw buffer resources and cross-lane sums of lane groups.
#pragma once

#include <hip/hip_runtime.h>

namespace fly {

constexpr int kBufferWord3 = 0x00020000;  // gfx9 raw buffer resource: 32-bit data, no swizzle

// A raw buffer of `bytes` bytes at p: loads at offsets past the end read zeros instead of faulting.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_of(const void *p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes, kBufferWord3);
}

// Sum of v over the lanes l, l + LPG, l + 2 LPG, ... of the wave, exact in lanes 0 .. LPG-1: a DPP
// rotation inside 16-lane rows for the stride of 8, then the permlane swaps across 16- and 32-lane halves
// (the swapped-in half of the source register holds the partner lanes).  Pairs add in the same order as
// a butterfly over strides 8, 16, 32.
template <int LPG>
__device__ __forceinline__ float group_sum(float v) {
  static_assert(LPG == 8 || LPG == 16 || LPG == 32, "lane groups of 8, 16 or 32");
  if constexpr (LPG == 8)
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128 /* row_ror:8 */, 0xF, 0xF, false));
  if constexpr (LPG <= 16)
    v += __int_as_float(__builtin_amdgcn_permlane16_swap(__float_as_int(v), __float_as_int(v), false, false)[1]);
  v += __int_as_float(__builtin_amdgcn_permlane32_swap(__float_as_int(v), __float_as_int(v), false, false)[1]);
  return v;
}

}  // namespace fly
