// The sparse products of training, float32 (chessfly/brain.py:66-99, _SparseRecurrent):
//   fly_spmm:   y = A x for A in CSR and x (cols, ldx) batch-fastest.  With the transposed structure of A
//               it is also grad_x = A^T grad_y.
//   fly_sddmm:  dL/dw_e = sum_b g[row_e, b] x[col_e, b] for every non-zero e of A, in CSR order.
// Gathers go through raw buffer resources: a 24-bit multiply-add gives the offset, and reads past a buffer
// return zeros, so indices from the caller can never make a kernel read out of bounds.
#include "common.hpp"
#include "device.hpp"

namespace fly {
namespace {

struct SpmmArgs {
  const int32_t *rowptr;  // nrows + 1
  const int32_t *col;     // nnz, column of each non-zero
  const float *val;       // nnz
  const float *x;         // (ncols, ldx)
  float *y;               // (nrows, ldy)
  int64_t ldx, ldy;
  uint32_t xbytes;        // ncols * ldx * 4, below 2^31
  int32_t nrows, batch, chunks;
};

// Wave -> (row, chunk of LPG * V columns), chunks outermost so one chunk is swept over every row before the
// next starts.  Lane group g gathers non-zero e0 + j * G + g; the groups' partial sums meet in group 0.
template <int G, int V, int UNROLL>
__global__ __launch_bounds__(256) void k_spmm(const SpmmArgs a) {
  constexpr int LPG = 64 / G;
  const uint32_t wave = blockIdx.x * 4u + (uint32_t)__builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t chunk = wave / (uint32_t)a.nrows, row = wave - chunk * (uint32_t)a.nrows;
  if (chunk >= (uint32_t)a.chunks) return;
  const int lane = threadIdx.x & 63, g = lane / LPG, s = lane % LPG;
  const int64_t col0 = (int64_t)chunk * (LPG * V) + (int64_t)s * V;

  float acc[V];
#pragma unroll
  for (int i = 0; i < V; ++i) acc[i] = 0.0f;
  const int32_t beg = a.rowptr[row], end = a.rowptr[row + 1];
  const int32_t n = end - beg;
  const __amdgpu_buffer_rsrc_t rc = buffer_of(a.col + beg, (uint32_t)n * 4u);
  const __amdgpu_buffer_rsrc_t rv = buffer_of(a.val + beg, (uint32_t)n * 4u);
  const __amdgpu_buffer_rsrc_t rx = buffer_of(a.x, a.xbytes);
  const uint32_t row_bytes = (uint32_t)a.ldx * 4u, voff = (uint32_t)col0 * 4u;
  for (int32_t e0 = 0; e0 < n; e0 += G * UNROLL) {
    int32_t c[UNROLL];
    float w[UNROLL];
#pragma unroll
    for (int j = 0; j < UNROLL; ++j) {   // past the row's end: column 0, weight 0
      const int off = (e0 + j * G + g) * 4;
      c[j] = (int32_t)__builtin_amdgcn_raw_buffer_load_b32(rc, off, 0, 0);
      w[j] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rv, off, 0, 0));
    }
    float xv[UNROLL][V];
#pragma unroll
    for (int j = 0; j < UNROLL; ++j) {
      const int o = (int)(__umul24((uint32_t)c[j], row_bytes) + voff);
      if constexpr (V == 4) {
        typedef unsigned u4 __attribute__((ext_vector_type(4)));
        const u4 v = __builtin_amdgcn_raw_buffer_load_b128(rx, o, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) xv[j][i] = __uint_as_float(v[i]);
      } else {
        xv[j][0] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rx, o, 0, 0));
      }
    }
#pragma unroll
    for (int j = 0; j < UNROLL; ++j)
#pragma unroll
      for (int i = 0; i < V; ++i) acc[i] = fmaf(w[j], xv[j][i], acc[i]);
  }
  if constexpr (G > 1) {
#pragma unroll
    for (int i = 0; i < V; ++i) acc[i] = group_sum<LPG>(acc[i]);
  }
  if (g != 0 || col0 >= a.batch) return;
  float *dst = a.y + (int64_t)row * a.ldy + col0;
  if constexpr (V == 4) {
    if (col0 + 4 <= a.batch) {
      *reinterpret_cast<float4 *>(dst) = make_float4(acc[0], acc[1], acc[2], acc[3]);
      return;
    }
  }
#pragma unroll
  for (int i = 0; i < V; ++i)
    if (col0 + i < a.batch) dst[i] = acc[i];
}

struct SddmmArgs {
  const int32_t *rowptr, *col;
  const float *g;  // (nrows, ldg)
  const float *x;  // (ncols, ldx)
  float *out;      // nnz
  int64_t ldg, ldx;
  uint32_t xbytes;
  int32_t nrows, batch;
};

// One wave per row, one lane per non-zero (64 at a time): lane e walks x[col_e, :] in 16-byte steps, 8 of
// them (one 128-byte line) per iteration, against g[row, :], which is wave-uniform and comes through the
// scalar cache.  No cross-lane sums.
template <int V>
__global__ __launch_bounds__(256) void k_sddmm(const SddmmArgs a) {
  constexpr int UNROLL = 8;
  const uint32_t row = blockIdx.x * 4u + (uint32_t)__builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (row >= (uint32_t)a.nrows) return;
  const int lane = threadIdx.x & 63;
  const int32_t beg = a.rowptr[row], end = a.rowptr[row + 1];
  const __amdgpu_buffer_rsrc_t rx = buffer_of(a.x, a.xbytes);
  // g is read-only for the kernel's lifetime: through the constant address space its uniform reads become
  // scalar loads instead of 64 identical vector reads
  typedef const __attribute__((address_space(4))) float cfloat;
  cfloat *grow = (cfloat *)(a.g + (int64_t)row * a.ldg);
  const uint32_t row_bytes = (uint32_t)a.ldx * 4u;
  constexpr int STEP = V * UNROLL;
  const int32_t full = a.batch / STEP * STEP;
  for (int32_t e0 = beg; e0 < end; e0 += 64) {
    const int32_t e = e0 + lane;
    const bool live = e < end;
    const uint32_t base = __umul24(live ? (uint32_t)a.col[e] : 0u, row_bytes);
    float acc = 0.0f;
    for (int32_t b = 0; b < full; b += STEP) {
      float xv[UNROLL][V];
#pragma unroll
      for (int j = 0; j < UNROLL; ++j) {
        const int o = (int)(base + (uint32_t)(b + j * V) * 4u);
        if constexpr (V == 4) {
          typedef unsigned u4 __attribute__((ext_vector_type(4)));
          const u4 v = __builtin_amdgcn_raw_buffer_load_b128(rx, o, 0, 0);
#pragma unroll
          for (int i = 0; i < 4; ++i) xv[j][i] = __uint_as_float(v[i]);
        } else {
          xv[j][0] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rx, o, 0, 0));
        }
      }
#pragma unroll
      for (int j = 0; j < UNROLL; ++j)
#pragma unroll
        for (int i = 0; i < V; ++i) acc = fmaf(grow[b + j * V + i], xv[j][i], acc);
    }
    for (int32_t b = full; b < a.batch; ++b)
      acc = fmaf(grow[b], __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rx, (int)(base + (uint32_t)b * 4u), 0, 0)),
                 acc);
    if (live) a.out[e] = acc;
  }
}

bool vec4_ok(const void *p, int64_t ld) { return ld % 4 == 0 && aligned(p, 16); }

uint32_t checked_bytes(int64_t rows, int64_t ld) {
  const int64_t bytes = rows * ld * 4;
  FLY_REQUIRE(bytes <= (int64_t)INT32_MAX, "the gathered operand must be below 2 GiB");
  return (uint32_t)std::max<int64_t>(bytes, 0);
}

template <int G, int V>
void launch_spmm(const SpmmArgs &a, hipStream_t st) {
  const int64_t waves = (int64_t)a.nrows * a.chunks;
  FLY_REQUIRE(waves < (int64_t)UINT32_MAX / 2, "spmm grid too large");
  hipLaunchKernelGGL((k_spmm<G, V, 4>), dim3(blocks_for(waves, 4)), dim3(256), 0, st, a);
}

}  // namespace
}  // namespace fly

using namespace fly;

extern "C" int fly_spmm(const int32_t *rowptr, const int32_t *col, const float *val, int64_t nrows, int64_t ncols,
                        const float *x, int64_t ldx, int64_t batch, float *y, int64_t ldy, void *stream) {
  return guard([&] {
    FLY_REQUIRE(nrows >= 0 && ncols >= 0 && batch >= 0, "negative size");
    FLY_REQUIRE(nrows < (int64_t)1 << 24 && ncols < (int64_t)1 << 24, "more than 2^24 rows or columns");
    if (!nrows || !batch) return;
    FLY_REQUIRE(rowptr && y && ldy >= batch, "bad argument");
    FLY_REQUIRE(ncols == 0 || (col && val && x && ldx >= batch && ldx < (1 << 22)), "bad argument");
    LaunchTimer timer(FLY_K_OTHER, as_stream(stream));
    SpmmArgs a{rowptr, col, val, x, y, ldx, ldy, checked_bytes(ncols, ldx), (int32_t)nrows, (int32_t)batch, 0};
    if (ncols == 0) a.xbytes = 0;   // every gather reads zeros: y = 0
    // 16-byte lanes in groups of 16 (64 columns per chunk) when the rows allow them, else 4-byte lanes in
    // groups of 8
    if (batch >= 4 && vec4_ok(x, ldx) && vec4_ok(y, ldy)) {
      a.chunks = (int32_t)((batch + 63) / 64);
      launch_spmm<4, 4>(a, as_stream(stream));
    } else {
      a.chunks = (int32_t)((batch + 7) / 8);
      launch_spmm<8, 1>(a, as_stream(stream));
    }
    check_launch("spmm");
  });
}

extern "C" int fly_sddmm(const int32_t *rowptr, const int32_t *col, int64_t nrows, int64_t ncols, const float *g,
                         int64_t ldg, const float *x, int64_t ldx, int64_t batch, float *out, void *stream) {
  return guard([&] {
    FLY_REQUIRE(nrows >= 0 && ncols >= 0 && batch >= 0, "negative size");
    FLY_REQUIRE(nrows < (int64_t)1 << 24 && ncols < (int64_t)1 << 24, "more than 2^24 rows or columns");
    if (!nrows) return;
    FLY_REQUIRE(rowptr && col && out && g && ldg >= batch, "bad argument");
    FLY_REQUIRE(ncols == 0 || (x && ldx >= batch && ldx < (1 << 22)), "bad argument");
    LaunchTimer timer(FLY_K_OTHER, as_stream(stream));
    SddmmArgs a{rowptr, col, g, x, out, ldg, ldx, ncols ? checked_bytes(ncols, ldx) : 0u, (int32_t)nrows,
                (int32_t)batch};
    const dim3 grid(blocks_for(nrows, 4)), block(256);
    if (batch >= 4 && vec4_ok(x, ldx))
      hipLaunchKernelGGL(k_sddmm<4>, grid, block, 0, as_stream(stream), a);
    else
      hipLaunchKernelGGL(k_sddmm<1>, grid, block, 0, as_stream(stream), a);
    check_launch("sddmm");
  });
}
