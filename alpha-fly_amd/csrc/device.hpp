// Device helpers shared by the kernels: raw buffer resources and cross-lane sums of lane groups.
#pragma once

#include <hip/hip_runtime.h>

#include <type_traits>
#include <utility>

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

// f(std::integral_constant<int, 0>) ... f(std::integral_constant<int, N - 1>), unrolled at compile time.
template <typename F, int... I>
__device__ __forceinline__ void static_for_seq(F &&f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F &&f) {
  static_for_seq(f, std::make_integer_sequence<int, N>{});
}

// Lane J of each group of N consecutive lanes (N = 8 or 16), to every lane of the group: ds_swizzle in bit mode,
// where lane l reads lane (l & (0x1F & ~(N - 1))) | J of its half-wave.  Cross-lane traffic of the LDS unit, not
// a memory access: a record loaded once per group reaches all of its lanes.
template <int N, int J>
__device__ __forceinline__ int group_bcast(int v) {
  static_assert((N == 8 || N == 16) && J >= 0 && J < N, "groups of 8 or 16 lanes");
  return __builtin_amdgcn_ds_swizzle(v, (0x1F & ~(N - 1)) | (J << 5));
}

// v from the lane (l ^ X) of lane l's group of 32 (X < 8 stays inside groups of 8): ds_swizzle in bit mode.
template <int X>
__device__ __forceinline__ float lane_xor(float v) {
  static_assert(X > 0 && X < 32, "xor mask of 5 bits");
  return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x1F | (X << 10)));
}

// Reduce-scatter inside each group of 8 lanes: d[r] holds a lane's share of value r (r = 0..7); lane s of the group
// returns the sum of value s over the group's 8 lanes.  Three halving exchanges (lanes 4 apart, 2, 1), 7 swizzles in
// all, summed in a fixed tree order.
__device__ __forceinline__ float group_reduce_scatter8(const float (&d)[8], int s) {
  const bool h4 = s & 4, h2 = s & 2, h1 = s & 1;
  float e[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) e[k] = (h4 ? d[k + 4] : d[k]) + lane_xor<4>(h4 ? d[k] : d[k + 4]);
  float f[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) f[k] = (h2 ? e[k + 2] : e[k]) + lane_xor<2>(h2 ? e[k] : e[k + 2]);
  return (h1 ? f[1] : f[0]) + lane_xor<1>(h1 ? f[0] : f[1]);
}

}  // namespace fly
