// What the search's evaluate callable hands back per batch (chessfly/model.py:120-128): the expected
// value of every board, and either the whole policy in half precision (lazy search) or the logits of the
// legal moves (eager search).  One pass over the logits, so only the requested bytes leave the card.
#include "common.hpp"

namespace fly {
namespace {

constexpr int kThreads = 256;
constexpr unsigned kMaxBlocks = 4096;  // grid-stride beyond 16 blocks per CU

__global__ void k_clear_flag(int32_t *flag) { *flag = 0; }

// P(win) - P(loss) under softmax(wdl[b]) (model.py:107-110): max-shifted exponentials, as softmax does.
__device__ inline float expected_value(const float *__restrict__ wdl, int64_t b) {
  const float w0 = wdl[3 * b], w1 = wdl[3 * b + 1], w2 = wdl[3 * b + 2];
  const float m = fmaxf(fmaxf(w0, w1), w2);
  const float e0 = expf(w0 - m), e1 = expf(w1 - m), e2 = expf(w2 - m);
  const float s = e0 + e1 + e2;
  return e0 / s - e2 / s;
}

// Lazy search: logits16 = half(logits), round to nearest even; four values per lane when `vec4`.
__global__ __launch_bounds__(kThreads) void k_lazy_outputs(const float *__restrict__ logits,
                                                           const float *__restrict__ wdl, int64_t batch,
                                                           int64_t total, bool vec4, _Float16 *__restrict__ out16,
                                                           float *__restrict__ values) {
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  const int64_t first = blockIdx.x * (int64_t)kThreads + threadIdx.x;
  for (int64_t b = first; b < batch; b += stride) values[b] = expected_value(wdl, b);
  if (vec4) {
    const float4 *src = reinterpret_cast<const float4 *>(logits);
    typedef _Float16 half4 __attribute__((ext_vector_type(4)));
    half4 *dst = reinterpret_cast<half4 *>(out16);
    for (int64_t i = first; i < total / 4; i += stride) {
      const float4 v = src[i];
      half4 h;
      h.x = static_cast<_Float16>(v.x);
      h.y = static_cast<_Float16>(v.y);
      h.z = static_cast<_Float16>(v.z);
      h.w = static_cast<_Float16>(v.w);
      dst[i] = h;
    }
  } else {
    for (int64_t i = first; i < total; i += stride) out16[i] = static_cast<_Float16>(logits[i]);
  }
}

// Eager search: legal[m] = logits[rows[m], cols[m]], indices wrapped as torch wraps negative ones; an
// index outside the shape yields NaN and raises the flag instead of reading out of bounds.
__global__ __launch_bounds__(kThreads) void k_legal_outputs(const float *__restrict__ logits,
                                                            const float *__restrict__ wdl, int64_t batch,
                                                            int64_t n_moves, const int64_t *__restrict__ rows,
                                                            const int64_t *__restrict__ cols, int64_t n_legal,
                                                            float *__restrict__ legal, float *__restrict__ values,
                                                            int32_t *__restrict__ bad) {
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  const int64_t first = blockIdx.x * (int64_t)kThreads + threadIdx.x;
  for (int64_t b = first; b < batch; b += stride) values[b] = expected_value(wdl, b);
  for (int64_t m = first; m < n_legal; m += stride) {
    int64_t r = rows[m], c = cols[m];
    r += r < 0 ? batch : 0;
    c += c < 0 ? n_moves : 0;
    if (r >= 0 && r < batch && c >= 0 && c < n_moves) {
      legal[m] = logits[r * n_moves + c];
    } else {
      legal[m] = __builtin_nanf("");
      atomicOr(bad, 1);
    }
  }
}

unsigned grid_for(int64_t work) {
  return std::max(1u, std::min<unsigned>(kMaxBlocks, blocks_for(std::max<int64_t>(work, 1), kThreads)));
}

// dst (pinned host memory, through its device address) = src (device memory), by a few workgroups that stride
// over 16-byte pieces and then the tail bytes.  Stores to host memory wait on the bus, and a CU's memory pipeline
// is in order: a full grid would stall every CU's other work behind them for the whole transfer, so only
// `gridDim.x` CUs carry it while the next batch's forward runs on the rest.
__global__ __launch_bounds__(kThreads) void k_host_copy(const uint8_t *__restrict__ src, uint8_t *__restrict__ dst,
                                                        int64_t bytes) {
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  const int64_t first = blockIdx.x * (int64_t)kThreads + threadIdx.x;
  const int64_t n16 = bytes / 16;
  const uint4 *s16 = reinterpret_cast<const uint4 *>(src);
  uint4 *d16 = reinterpret_cast<uint4 *>(dst);
  for (int64_t i = first; i < n16; i += stride) d16[i] = s16[i];
  for (int64_t i = n16 * 16 + first; i < bytes; i += stride) dst[i] = src[i];
}

}  // namespace
}  // namespace fly

using namespace fly;

extern "C" int fly_evaluator_outputs(const float *logits, const float *wdl, int64_t batch, int64_t n_moves,
                                     const int64_t *rows, const int64_t *cols, int64_t n_legal, void *logits16,
                                     float *legal, float *values, int32_t *bad, void *stream) {
  return guard([&] {
    FLY_REQUIRE(batch >= 0 && n_moves >= 0 && n_legal >= 0, "negative size");
    FLY_REQUIRE(bad != nullptr, "the index flag pointer is null");
    FLY_REQUIRE(!batch || (wdl && values), "wdl and values are required for a non-empty batch");
    hipStream_t st = as_stream(stream);
    hipLaunchKernelGGL(k_clear_flag, dim3(1), dim3(1), 0, st, bad);
    check_launch("index flag");
    if (rows == nullptr) {
      const int64_t total = batch * n_moves;
      FLY_REQUIRE(!total || (logits && logits16), "logits and logits16 are required for the lazy outputs");
      if (!batch) return;
      const bool vec4 = total % 4 == 0 && aligned(logits, 16) && aligned(logits16, 8);
      hipLaunchKernelGGL(k_lazy_outputs, dim3(grid_for(std::max(vec4 ? total / 4 : total, batch))), dim3(kThreads),
                         0, st, logits, wdl, batch, total, vec4, static_cast<_Float16 *>(logits16), values);
      check_launch("lazy outputs");
    } else {
      FLY_REQUIRE(!n_legal || (cols && legal), "cols and legal are required for the legal-move gather");
      FLY_REQUIRE(!n_legal || (logits && batch && n_moves), "legal moves requested from an empty policy");
      if (!batch && !n_legal) return;
      hipLaunchKernelGGL(k_legal_outputs, dim3(grid_for(std::max(n_legal, batch))), dim3(kThreads), 0, st, logits,
                         wdl, batch, n_moves, rows, cols, n_legal, legal, values, bad);
      check_launch("legal outputs");
    }
  });
}

extern "C" int fly_evaluator_download(const void *src, void *dst_host, size_t bytes, int32_t workgroups,
                                      void *stream) {
  return guard([&] {
    if (bytes == 0) return;
    FLY_REQUIRE(src != nullptr && dst_host != nullptr, "null pointer");
    FLY_REQUIRE(aligned(src, 16) && aligned(dst_host, 16), "source and destination must be 16-byte aligned");
    hipPointerAttribute_t sattr{};
    const hipError_t se = hipPointerGetAttributes(&sattr, src);
    if (se != hipSuccess) (void)hipGetLastError();   // an unknown pointer: clear the error, report it below
    FLY_REQUIRE(se == hipSuccess && (sattr.type == hipMemoryTypeDevice || sattr.type == hipMemoryTypeManaged),
                "the source must be device memory");
    hipPointerAttribute_t attr{};
    const hipError_t e = hipPointerGetAttributes(&attr, dst_host);
    if (e != hipSuccess) (void)hipGetLastError();
    FLY_REQUIRE(e == hipSuccess && attr.type == hipMemoryTypeHost && attr.devicePointer != nullptr,
                "the destination must be pinned host memory (hipHostMalloc, torch pin_memory=True)");
    const int tuned = tuning_snapshot().download_blocks;
    const int wg = workgroups > 0 ? workgroups : (tuned > 0 ? tuned : 16);
    const int64_t pieces = (int64_t)((bytes + 15) / 16);
    const unsigned grid = (unsigned)std::max<int64_t>(1, std::min<int64_t>(wg, (pieces + kThreads - 1) / kThreads));
    // the device address of dst_host itself, whether the runtime reports the allocation's base or the pointer's own
    // addresses (they then differ by the same offset)
    uint8_t *dst = static_cast<uint8_t *>(attr.devicePointer);
    if (attr.hostPointer != nullptr) dst += static_cast<uint8_t *>(dst_host) - static_cast<uint8_t *>(attr.hostPointer);
    hipLaunchKernelGGL(k_host_copy, dim3(grid), dim3(kThreads), 0, as_stream(stream), static_cast<const uint8_t *>(src),
                       dst, (int64_t)bytes);
    check_launch("download");
  });
}
