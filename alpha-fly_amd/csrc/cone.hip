// Light cone on the device: reach masks, compaction into sorted row lists, and the per-step
// sub-matrices A_t = W[R_t, R_{t-1}] in W's edge order.  Integer work only; every kernel is
// deterministic (order-preserving scans, row-parallel fills), so the result is bit-exact with the
// definition in chessfly/brain.py:126-173 (LightCone) and :102-123 (_SubMatrix).
#include "common.hpp"
#include "sweep.hpp"

namespace fly {
namespace {

constexpr int kScanThreads = 1024;

// bad |= any index outside [0, n)
__global__ void k_check_index(const int32_t *__restrict__ idx, int64_t k, int64_t n, int32_t *__restrict__ bad) {
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i < k) {
    const int32_t v = idx[i];
    if (v < 0 || v >= n) atomicOr(bad, 1);
  }
}

// CSR sanity: crow[0] == 0, crow non-decreasing, crow[n] == n_edges (bit 2); pre in range via k_check_index.
__global__ void k_check_crow(const int32_t *__restrict__ crow, int64_t n, int64_t n_edges, int32_t *__restrict__ bad) {
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i < n) {
    if (crow[i] > crow[i + 1]) atomicOr(bad, 2);
    if (i == 0 && crow[0] != 0) atomicOr(bad, 2);
    if (i == n - 1 && crow[n] != n_edges) atomicOr(bad, 2);
  }
}

__global__ void k_fill_u8(uint8_t *__restrict__ m, uint8_t v, int64_t n) {
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i < n) m[i] = v;
}

__global__ void k_fill_i32(int32_t *__restrict__ m, int32_t v, int64_t n) {
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i < n) m[i] = v;
}

__global__ void k_mark(uint8_t *__restrict__ m, const int32_t *__restrict__ idx, int64_t k) {
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i < k) m[idx[i]] = 1;
}

// pos[idx[j]] = j; with repeated ids the largest j wins (what a sequential assignment leaves).
__global__ void k_positions(int32_t *__restrict__ pos, const int32_t *__restrict__ idx, int64_t k) {
  const int64_t j = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (j < k) atomicMax(&pos[idx[j]], (int32_t)j);
}

// V_t[r] = V_{t-1}[r] or any presynaptic partner of r is in V_{t-1}   (row-parallel, no races)
__global__ void k_grow_forward(const int32_t *__restrict__ crow, const int32_t *__restrict__ pre,
                               const uint8_t *__restrict__ vin, uint8_t *__restrict__ vout, int64_t n) {
  const int64_t r = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (r >= n) return;
  uint8_t v = vin[r];
  if (!v) {
    const int32_t end = crow[r + 1];
    for (int32_t e = crow[r]; e < end; ++e)
      if (vin[pre[e]]) { v = 1; break; }
  }
  vout[r] = v;
}

// D_t |= presynaptic partners of D_{t+1} rows.  dout already holds a copy of din; concurrent stores all
// write 1, so the result does not depend on their order.  16 lanes per row, lane s marking the partners s, s + 16,
// ..., so a hub row's thousands of partners do not fall to one lane.
__global__ __launch_bounds__(256) void k_grow_backward(const int32_t *__restrict__ crow, const int32_t *__restrict__ pre,
                                                       const uint8_t *__restrict__ din, uint8_t *__restrict__ dout,
                                                       int64_t n) {
  const int s = threadIdx.x & 15;
  const int64_t r = blockIdx.x * 16 + (threadIdx.x >> 4);
  if (r >= n || !din[r]) return;
  const int32_t end = crow[r + 1];
  for (int32_t e = crow[r] + s; e < end; e += 16) dout[pre[e]] = 1;
}

// Block-wide inclusive scan of one value per thread (kScanThreads threads).
__device__ int32_t block_inclusive_scan(int32_t v, int32_t *part) {
  const int tid = threadIdx.x;
  part[tid] = v;
  __syncthreads();
  for (int off = 1; off < kScanThreads; off <<= 1) {
    const int32_t add = tid >= off ? part[tid - off] : 0;
    __syncthreads();
    part[tid] += add;
    __syncthreads();
  }
  return part[tid];
}

// Multi-workgroup order-preserving compaction and scan: a workgroup owns a tile of kTile indices, thread j the
// 8 consecutive indices [8j, 8j + 8) of it, so positions follow index order.  Three passes: per-tile totals,
// one single-workgroup scan of those (k_scan), then per-tile positions from the tile's offset.
constexpr int kPer = 8, kTile = kScanThreads * kPer;

__device__ __forceinline__ int64_t tile_base() { return (int64_t)blockIdx.x * kTile + (int64_t)threadIdx.x * kPer; }

__global__ __launch_bounds__(kScanThreads) void k_tile_flags(const uint8_t *__restrict__ a, const uint8_t *__restrict__ b,
                                                             int64_t n, int32_t *__restrict__ tile_sum) {
  __shared__ int32_t part[kScanThreads];
  const int64_t base = tile_base();
  int32_t c = 0;
#pragma unroll
  for (int k = 0; k < kPer; ++k) c += (base + k < n && a[base + k] && b[base + k]) ? 1 : 0;
  const int32_t incl = block_inclusive_scan(c, part);
  if (threadIdx.x == kScanThreads - 1) tile_sum[blockIdx.x] = incl;
}

// rows = sorted {i : a[i] && b[i]}, where[i] = position in rows or -1
__global__ __launch_bounds__(kScanThreads) void k_tile_compact(const uint8_t *__restrict__ a,
                                                               const uint8_t *__restrict__ b, int64_t n,
                                                               const int32_t *__restrict__ tile_off,
                                                               int32_t *__restrict__ rows, int32_t *__restrict__ where) {
  __shared__ int32_t part[kScanThreads];
  const int64_t base = tile_base();
  int32_t c = 0;
#pragma unroll
  for (int k = 0; k < kPer; ++k) c += (base + k < n && a[base + k] && b[base + k]) ? 1 : 0;
  const int32_t incl = block_inclusive_scan(c, part);
  int32_t run = tile_off[blockIdx.x] + incl - c;
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int64_t i = base + k;
    if (i >= n) break;
    if (a[i] && b[i]) {
      rows[run] = (int32_t)i;
      where[i] = run++;
    } else {
      where[i] = -1;
    }
  }
}

__global__ __launch_bounds__(kScanThreads) void k_tile_sums(const int32_t *__restrict__ in, int64_t n,
                                                            int32_t *__restrict__ tile_sum) {
  __shared__ int32_t part[kScanThreads];
  const int64_t base = tile_base();
  int32_t c = 0;
#pragma unroll
  for (int k = 0; k < kPer; ++k) c += base + k < n ? in[base + k] : 0;
  const int32_t incl = block_inclusive_scan(c, part);
  if (threadIdx.x == kScanThreads - 1) tile_sum[blockIdx.x] = incl;
}

// out[i] = sum of in[0..i) from the tile offsets; the last tile also writes out[n] = total
__global__ __launch_bounds__(kScanThreads) void k_tile_scan(const int32_t *__restrict__ in, int64_t n,
                                                            const int32_t *__restrict__ tile_off, int64_t ntiles,
                                                            int32_t *__restrict__ out) {
  __shared__ int32_t part[kScanThreads];
  const int64_t base = tile_base();
  int32_t c = 0;
#pragma unroll
  for (int k = 0; k < kPer; ++k) c += base + k < n ? in[base + k] : 0;
  const int32_t incl = block_inclusive_scan(c, part);
  int32_t run = tile_off[blockIdx.x] + incl - c;
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int64_t i = base + k;
    if (i >= n) break;
    out[i] = run;
    run += in[i];
  }
  if (blockIdx.x == ntiles - 1 && threadIdx.x == 0) out[n] = tile_off[ntiles];
}

// One workgroup: out[i] = sum of in[0..i), out[n] = total.
__global__ __launch_bounds__(kScanThreads) void k_scan(const int32_t *__restrict__ in, int64_t n, int32_t *__restrict__ out) {
  __shared__ int32_t part[kScanThreads];
  const int64_t seg = (n + kScanThreads - 1) / kScanThreads;
  const int64_t beg = min(n, (int64_t)threadIdx.x * seg), end = min(n, beg + seg);
  int32_t c = 0;
  for (int64_t i = beg; i < end; ++i) c += in[i];
  const int32_t incl = block_inclusive_scan(c, part);
  int32_t run = incl - c;
  for (int64_t i = beg; i < end; ++i) {
    out[i] = run;
    run += in[i];
  }
  if (threadIdx.x == kScanThreads - 1) out[n] = incl;
}

// prev[i] = position of R_t[i] in R_{t-1} (-1 if absent or R_{t-1} empty); usrc[i] = its input position.
__global__ void k_step_index(const int32_t *__restrict__ rows, int64_t nr, const int32_t *__restrict__ where_prev,
                             const int32_t *__restrict__ in_pos, int32_t *__restrict__ prev, int32_t *__restrict__ usrc) {
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i >= nr) return;
  const int32_t r = rows[i];
  prev[i] = where_prev ? where_prev[r] : -1;
  usrc[i] = in_pos[r];
}

// Per row of R_t (one wave each, lanes across the row's edges in W's order): how many of its presynaptic partners
// lie in R_{t-1}, and their local columns and edge ids, written in edge order from the lanes' ballot.
__global__ __launch_bounds__(256) void k_row_count(const int32_t *__restrict__ rows, int64_t nr,
                                                   const int32_t *__restrict__ crow, const int32_t *__restrict__ pre,
                                                   const int32_t *__restrict__ where_prev, int32_t *__restrict__ cnt) {
  const int64_t i = blockIdx.x * 4 + (int64_t)__builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (i >= nr) return;
  const int lane = threadIdx.x & 63;
  const int32_t r = rows[i], beg = crow[r], end = crow[r + 1];
  int32_t c = 0;
  for (int32_t e0 = beg; e0 < end; e0 += 64) {
    const int32_t e = e0 + lane;
    c += __popcll(__ballot(e < end && where_prev[pre[e]] >= 0));
  }
  if (lane == 0) cnt[i] = c;
}

__global__ __launch_bounds__(256) void k_row_fill(const int32_t *__restrict__ rows, int64_t nr,
                                                  const int32_t *__restrict__ crow, const int32_t *__restrict__ pre,
                                                  const int32_t *__restrict__ where_prev,
                                                  const int32_t *__restrict__ rowptr, int32_t *__restrict__ col,
                                                  int32_t *__restrict__ edge) {
  const int64_t i = blockIdx.x * 4 + (int64_t)__builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (i >= nr) return;
  const int lane = threadIdx.x & 63;
  const int32_t r = rows[i], beg = crow[r], end = crow[r + 1];
  const uint64_t below = (1ull << lane) - 1ull;
  int32_t p = rowptr[i];
  for (int32_t e0 = beg; e0 < end; e0 += 64) {
    const int32_t e = e0 + lane;
    const int32_t w = e < end ? where_prev[pre[e]] : -1;
    const uint64_t m = __ballot(w >= 0);
    if (w >= 0) {
      const int32_t pos = p + __popcll(m & below);
      col[pos] = w;
      edge[pos] = e;
    }
    p += __popcll(m);
  }
}

__global__ void k_lookup(const int32_t *__restrict__ table, const int32_t *__restrict__ idx, int64_t k,
                         int32_t *__restrict__ out) {
  const int64_t j = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (j < k) out[j] = table[idx[j]];
}

constexpr int kThreads = 256;

void copy_d2d(void *dst, const void *src, size_t bytes, hipStream_t st) {
  if (bytes) FLY_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, st));
}

// out[i] = sum of in[0..i), out[n] = total: one workgroup up to one tile, else the tile totals, their scan and
// the per-tile passes.  tile_sum and tile_off hold ceil(n / kTile) and one more entries.
void exclusive_scan(const int32_t *in, int64_t n, int32_t *out, int32_t *tile_sum, int32_t *tile_off, hipStream_t st) {
  if (n <= kTile) {
    hipLaunchKernelGGL(k_scan, dim3(1), dim3(kScanThreads), 0, st, in, n, out);
    return;
  }
  const int64_t ntiles = (n + kTile - 1) / kTile;
  hipLaunchKernelGGL(k_tile_sums, dim3((unsigned)ntiles), dim3(kScanThreads), 0, st, in, n, tile_sum);
  hipLaunchKernelGGL(k_scan, dim3(1), dim3(kScanThreads), 0, st, tile_sum, ntiles, tile_off);
  hipLaunchKernelGGL(k_tile_scan, dim3((unsigned)ntiles), dim3(kScanThreads), 0, st, in, n, tile_off, ntiles, out);
}

}  // namespace

void validate_graph(int64_t n, int64_t n_edges, const int32_t *crow, const int32_t *pre, hipStream_t st) {
  DevArray<int32_t> bad(1);
  hipLaunchKernelGGL(k_fill_i32, dim3(1), dim3(1), 0, st, bad.p, 0, (int64_t)1);
  hipLaunchKernelGGL(k_check_crow, dim3(blocks_for(n, kThreads)), dim3(kThreads), 0, st, crow, n, n_edges, bad.p);
  if (n_edges) hipLaunchKernelGGL(k_check_index, dim3(blocks_for(n_edges, kThreads)), dim3(kThreads), 0, st, pre, n_edges, n, bad.p);
  check_launch("graph validation");
  int32_t h = 0;
  FLY_HIP(hipMemcpyAsync(&h, bad.p, sizeof(h), hipMemcpyDeviceToHost, st));
  FLY_HIP(hipStreamSynchronize(st));
  FLY_REQUIRE(!(h & 2), "crow is not a CSR row pointer of n_edges edges (crow[0] == 0, non-decreasing, crow[n] == n_edges)");
  FLY_REQUIRE(!(h & 1), "pre holds a neuron id outside [0, n)");
}

}  // namespace fly

using namespace fly;

extern "C" int fly_cone_create(int64_t n, int64_t n_edges, const int32_t *crow, const int32_t *pre,
                               const int32_t *in_idx, int64_t n_in, const int32_t *out_idx, int64_t n_out,
                               int32_t steps, int32_t flags, void *stream, fly_cone **out) {
  return guard([&] {
    FLY_REQUIRE(out != nullptr, "out is null");
    *out = nullptr;
    FLY_REQUIRE(n > 0 && n < (int64_t)INT32_MAX, "n must be in [1, 2^31)");
    FLY_REQUIRE(n_edges >= 0 && n_edges < (int64_t)INT32_MAX, "n_edges must be in [0, 2^31)");
    FLY_REQUIRE(steps >= 0 && steps <= 64, "steps must be in [0, 64]");
    FLY_REQUIRE((flags & ~FLY_CONE_UNPRUNED) == 0, "unknown cone flag");
    FLY_REQUIRE(n_in >= 0 && n_out >= 0, "negative index count");
    FLY_REQUIRE(crow && (pre || n_edges == 0), "graph pointer is null");
    FLY_REQUIRE((in_idx || n_in == 0) && (out_idx || n_out == 0), "index pointer is null");
    hipStream_t st = as_stream(stream);
    validate_graph(n, n_edges, crow, pre, st);
    {
      DevArray<int32_t> bad(1);
      hipLaunchKernelGGL(k_fill_i32, dim3(1), dim3(1), 0, st, bad.p, 0, (int64_t)1);
      if (n_in) hipLaunchKernelGGL(k_check_index, dim3(blocks_for(n_in, kThreads)), dim3(kThreads), 0, st, in_idx, n_in, n, bad.p);
      if (n_out) hipLaunchKernelGGL(k_check_index, dim3(blocks_for(n_out, kThreads)), dim3(kThreads), 0, st, out_idx, n_out, n, bad.p);
      check_launch("index validation");
      int32_t h = 0;
      FLY_HIP(hipMemcpyAsync(&h, bad.p, sizeof(h), hipMemcpyDeviceToHost, st));
      FLY_HIP(hipStreamSynchronize(st));
      FLY_REQUIRE(h == 0, "in_idx or out_idx holds a neuron id outside [0, n)");
    }

    auto cone = std::make_unique<fly_cone>();
    cone->sweep_cache = std::make_shared<ConeSweepCache>();
    cone->device = current_device();
    cone->n = n;
    cone->n_edges = n_edges;
    cone->n_in = n_in;
    cone->n_out = n_out;
    cone->steps = steps;
    const int T = steps;
    const unsigned nb = blocks_for(n, kThreads);

    // Reach masks V_0..V_T and D_0..D_T.
    DevArray<uint8_t> fwd((size_t)(T + 1) * n), bwd((size_t)(T + 1) * n);
    auto V = [&](int t) { return fwd.p + (size_t)t * n; };
    auto D = [&](int t) { return bwd.p + (size_t)t * n; };
    hipLaunchKernelGGL(k_fill_u8, dim3(blocks_for((T + 1) * n, kThreads)), dim3(kThreads), 0, st, fwd.p, (uint8_t)0, (int64_t)(T + 1) * n);
    hipLaunchKernelGGL(k_fill_u8, dim3(blocks_for((T + 1) * n, kThreads)), dim3(kThreads), 0, st, bwd.p, (uint8_t)0, (int64_t)(T + 1) * n);
    if (flags & FLY_CONE_UNPRUNED) {  // every neuron varies from step 1 and every neuron matters
      if (T >= 1)
        hipLaunchKernelGGL(k_fill_u8, dim3(blocks_for(T * n, kThreads)), dim3(kThreads), 0, st, V(1), (uint8_t)1, (int64_t)T * n);
      hipLaunchKernelGGL(k_fill_u8, dim3(blocks_for((T + 1) * n, kThreads)), dim3(kThreads), 0, st, D(0), (uint8_t)1,
                         (int64_t)(T + 1) * n);
    } else {
      if (T >= 1 && n_in) hipLaunchKernelGGL(k_mark, dim3(blocks_for(n_in, kThreads)), dim3(kThreads), 0, st, V(1), in_idx, n_in);
      for (int t = 2; t <= T; ++t)
        hipLaunchKernelGGL(k_grow_forward, dim3(nb), dim3(kThreads), 0, st, crow, pre, V(t - 1), V(t), n);
      if (n_out) hipLaunchKernelGGL(k_mark, dim3(blocks_for(n_out, kThreads)), dim3(kThreads), 0, st, D(T), out_idx, n_out);
      for (int t = T - 1; t >= 0; --t) {
        copy_d2d(D(t), D(t + 1), (size_t)n, st);
        hipLaunchKernelGGL(k_grow_backward, dim3(blocks_for(n, 16)), dim3(256), 0, st, crow, pre, D(t + 1), D(t), n);
      }
    }
    check_launch("reach masks");

    // R_t = sorted(V_t & D_t) and the position tables where_t.
    std::vector<DevArray<int32_t>> where(T + 1);
    cone->rows.resize(T + 1);
    DevArray<int32_t> counts(T + 1);
    const int64_t ntiles = (n + kTile - 1) / kTile;
    DevArray<int32_t> tile_sum(ntiles), tile_off(ntiles + 1);
    for (int t = 0; t <= T; ++t) {
      where[t].alloc(n);
      cone->rows[t].alloc(n);
      hipLaunchKernelGGL(k_tile_flags, dim3((unsigned)ntiles), dim3(kScanThreads), 0, st, V(t), D(t), n, tile_sum.p);
      hipLaunchKernelGGL(k_scan, dim3(1), dim3(kScanThreads), 0, st, tile_sum.p, ntiles, tile_off.p);
      hipLaunchKernelGGL(k_tile_compact, dim3((unsigned)ntiles), dim3(kScanThreads), 0, st, V(t), D(t), n, tile_off.p,
                         cone->rows[t].p, where[t].p);
      copy_d2d(counts.p + t, tile_off.p + ntiles, sizeof(int32_t), st);
    }
    check_launch("row compaction");
    std::vector<int32_t> hcount(T + 1);
    FLY_HIP(hipMemcpyAsync(hcount.data(), counts.p, sizeof(int32_t) * (T + 1), hipMemcpyDeviceToHost, st));
    FLY_HIP(hipStreamSynchronize(st));
    cone->rows_n.assign(hcount.begin(), hcount.end());

    DevArray<int32_t> in_pos(n);
    hipLaunchKernelGGL(k_fill_i32, dim3(nb), dim3(kThreads), 0, st, in_pos.p, -1, n);
    if (n_in) hipLaunchKernelGGL(k_positions, dim3(blocks_for(n_in, kThreads)), dim3(kThreads), 0, st, in_pos.p, in_idx, n_in);

    // Per step: carried / input tables, and the counts and row pointers of A_t.
    cone->rowptr.resize(T + 1);
    cone->col.resize(T + 1);
    cone->edge.resize(T + 1);
    cone->prev.resize(T + 1);
    cone->usrc.resize(T + 1);
    cone->has_op.assign(T + 1, 0);
    cone->nnz.assign(T + 1, 0);
    DevArray<int32_t> cnt(n);
    for (int t = 1; t <= T; ++t) {
      const int64_t nr = cone->rows_n[t];
      cone->prev[t].alloc(nr);
      cone->usrc[t].alloc(nr);
      const bool op = cone->rows_n[t - 1] > 0;
      cone->has_op[t] = op ? 1 : 0;
      if (nr)
        hipLaunchKernelGGL(k_step_index, dim3(blocks_for(nr, kThreads)), dim3(kThreads), 0, st, cone->rows[t].p, nr,
                           op ? where[t - 1].p : nullptr, in_pos.p, cone->prev[t].p, cone->usrc[t].p);
      if (op) {
        cone->rowptr[t].alloc(nr + 1);
        if (nr)
          hipLaunchKernelGGL(k_row_count, dim3(blocks_for(nr, 4)), dim3(256), 0, st, cone->rows[t].p, nr, crow, pre,
                             where[t - 1].p, cnt.p);
        exclusive_scan(cnt.p, nr, cone->rowptr[t].p, tile_sum.p, tile_off.p, st);
        // read back nnz_t before the count buffer is reused by the next step
        int32_t h = 0;
        FLY_HIP(hipMemcpyAsync(&h, cone->rowptr[t].p + nr, sizeof(h), hipMemcpyDeviceToHost, st));
        FLY_HIP(hipStreamSynchronize(st));
        cone->nnz[t] = h;
        cone->col[t].alloc(h);
        cone->edge[t].alloc(h);
        if (nr && h)
          hipLaunchKernelGGL(k_row_fill, dim3(blocks_for(nr, 4)), dim3(256), 0, st, cone->rows[t].p, nr, crow, pre,
                             where[t - 1].p, cone->rowptr[t].p, cone->col[t].p, cone->edge[t].p);
      }
    }
    cone->out_src.alloc(n_out);
    cone->out_idx.alloc(n_out);
    if (n_out) {
      hipLaunchKernelGGL(k_lookup, dim3(blocks_for(n_out, kThreads)), dim3(kThreads), 0, st, where[T].p, out_idx, n_out,
                         cone->out_src.p);
      copy_d2d(cone->out_idx.p, out_idx, sizeof(int32_t) * n_out, st);
    }
    check_launch("sub-matrices");
    FLY_HIP(hipStreamSynchronize(st));
    *out = cone.release();
  });
}

extern "C" int fly_cone_destroy(fly_cone *cone) {
  return guard([&] { delete cone; });
}

extern "C" int fly_cone_sizes(const fly_cone *cone, int64_t *rows, int64_t *nnz, int32_t *has_op) {
  return guard([&] {
    FLY_REQUIRE(cone, "cone is null");
    for (int t = 0; t <= cone->steps; ++t) {
      if (rows) rows[t] = cone->rows_n[t];
      if (nnz) nnz[t] = cone->nnz[t];
      if (has_op) has_op[t] = cone->has_op[t];
    }
  });
}

extern "C" int fly_cone_rows(const fly_cone *cone, int32_t t, int32_t *rows, void *stream) {
  return guard([&] {
    FLY_REQUIRE(cone, "cone is null");
    FLY_REQUIRE(t >= 0 && t <= cone->steps, "step out of range");
    if (cone->rows_n[t] == 0) return;
    FLY_REQUIRE(rows, "rows is null");
    copy_d2d(rows, cone->rows[t].p, sizeof(int32_t) * cone->rows_n[t], as_stream(stream));
  });
}

extern "C" int fly_cone_step(const fly_cone *cone, int32_t t, int32_t *crow, int32_t *col, int32_t *edge,
                             int32_t *prev, int32_t *usrc, void *stream) {
  return guard([&] {
    FLY_REQUIRE(cone, "cone is null");
    FLY_REQUIRE(t >= 1 && t <= cone->steps, "step out of range");
    hipStream_t st = as_stream(stream);
    const int64_t nr = cone->rows_n[t];
    if (cone->has_op[t]) {
      if (crow) copy_d2d(crow, cone->rowptr[t].p, sizeof(int32_t) * (nr + 1), st);
      if (col) copy_d2d(col, cone->col[t].p, sizeof(int32_t) * cone->nnz[t], st);
      if (edge) copy_d2d(edge, cone->edge[t].p, sizeof(int32_t) * cone->nnz[t], st);
    }
    if (prev) copy_d2d(prev, cone->prev[t].p, sizeof(int32_t) * nr, st);
    if (usrc) copy_d2d(usrc, cone->usrc[t].p, sizeof(int32_t) * nr, st);
  });
}

extern "C" int fly_cone_outputs(const fly_cone *cone, int32_t *out_src, void *stream) {
  return guard([&] {
    FLY_REQUIRE(cone, "cone is null");
    if (cone->n_out == 0) return;
    FLY_REQUIRE(out_src, "out_src is null");
    copy_d2d(out_src, cone->out_src.p, sizeof(int32_t) * cone->n_out, as_stream(stream));
  });
}
