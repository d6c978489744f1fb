// Measurement only: the ceiling of the state step's memory access pattern on this GPU.  A wave splits into
// G groups of 64 / G lanes; per round group g reads the first 1024 / G bytes of row idx[e + g] (16 bytes per
// lane) and folds them into one register with 4 adds (the step spends 8 FMAs).  G = 8 (128 bytes per row) is
// exactly the gather of the state step's 64-column chunks; G = 16 (64 bytes per row) is a half chunk, as the
// last chunk of a batch of 32 columns past a multiple of 64.  Timing it over working sets that fit the L2, the
// Infinity Cache or neither gives the random-row gather rate the state step can at best reach.
#include "common.hpp"
#include "device.hpp"

namespace fly {
namespace {

constexpr int kRoundsPerWave = 64;

template <int G>
__global__ __launch_bounds__(256) void k_gather_probe(const char *base, uint32_t bytes, uint32_t row_bytes,
                                                      const int32_t *__restrict__ idx, int64_t n,
                                                      float *__restrict__ sink) {
  constexpr int LPG = 64 / G;
  const int lane = threadIdx.x & 63, g = lane / LPG, s = lane % LPG;
  const int64_t wave = blockIdx.x * 4ll + (threadIdx.x >> 6);
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<char *>(base), (short)0,
                                                                     (int)bytes, kBufferWord3);
  float acc = 0.0f;
  const int64_t first = wave * kRoundsPerWave * G;
#pragma unroll 4
  for (int k = 0; k < kRoundsPerWave; ++k) {
    const int64_t e = first + k * G + g;
    if (e >= n) break;
    // offsets past the buffer read zeros: every access stays in bounds whatever idx holds
    const uint32_t off = __umul24((uint32_t)idx[e], row_bytes) + (uint32_t)s * 16u;
    typedef unsigned u4 __attribute__((ext_vector_type(4)));
    const u4 v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
    acc += __uint_as_float(v.x) + __uint_as_float(v.y) + __uint_as_float(v.z) + __uint_as_float(v.w);
  }
  if (acc == 1234.5f) sink[threadIdx.x] = acc;  // keeps the loads alive; a probe over zeros never stores
}

}  // namespace
}  // namespace fly

using namespace fly;

extern "C" int fly_gather_probe(const void *base, int64_t bytes, int64_t row_bytes, int64_t read_bytes,
                                const int32_t *idx, int64_t n, float *sink, void *stream) {
  return guard([&] {
    FLY_REQUIRE(base && idx && sink, "null argument");
    FLY_REQUIRE(bytes > 0 && bytes <= INT32_MAX, "the probed buffer must hold 1 .. 2^31-1 bytes");
    FLY_REQUIRE(read_bytes == 64 || read_bytes == 128, "read_bytes must be 64 or 128");
    FLY_REQUIRE(row_bytes >= read_bytes && row_bytes < (1 << 24), "row_bytes must be read_bytes .. 2^24-1");
    FLY_REQUIRE(n > 0 && n <= (int64_t)1 << 34, "n out of range");
    const int G = read_bytes == 128 ? 8 : 16;
    const int64_t waves = (n + kRoundsPerWave * G - 1) / (kRoundsPerWave * G);
    FLY_REQUIRE(waves < (int64_t)UINT32_MAX, "probe grid too large");
    LaunchTimer timer(FLY_K_OTHER, as_stream(stream));
    if (G == 8)
      hipLaunchKernelGGL(k_gather_probe<8>, dim3(blocks_for(waves, 4)), dim3(256), 0, as_stream(stream),
                         static_cast<const char *>(base), (uint32_t)bytes, (uint32_t)row_bytes, idx, n, sink);
    else
      hipLaunchKernelGGL(k_gather_probe<16>, dim3(blocks_for(waves, 4)), dim3(256), 0, as_stream(stream),
                         static_cast<const char *>(base), (uint32_t)bytes, (uint32_t)row_bytes, idx, n, sink);
    check_launch("gather probe");
  });
}
