// The sparse products of training, float32 (chessfly/brain.py:66-99, _SparseRecurrent):
//   fly_spmm:   y = A x for A in CSR and x (cols, ldx) batch-fastest.  With the transposed structure of A
//               it is also grad_x = A^T grad_y.
//   fly_sddmm:  dL/dw_e = sum_b g[row_e, b] x[col_e, b] for every non-zero e of A, in CSR order.
// Gathers go through raw buffer resources: a 24-bit multiply-add gives the offset, and reads past a buffer
// return zeros, so indices from the caller can never make a kernel read out of bounds.
#include "common.hpp"
#include "device.hpp"
#include "step_kernels.hpp"

namespace fly {
namespace {

struct SpmmArgs {
  const int32_t *rowptr;  // nrows + 1
  const int32_t *col;     // nnz, column of each non-zero
  const float *val;       // nnz values, or the vector val_ids index into
  const int32_t *val_ids; // null, or per non-zero the index of its value in val
  uint32_t val_bytes;     // bytes of val when val_ids is given (reads past it give 0)
  const float *x;         // (ncols, ldx)
  float *y;               // (nrows, ldy)
  int64_t ldx, ldy;
  uint32_t xbytes;        // ncols * ldx * 4, below 2^31
  int32_t nrows, batch, chunks;
  int32_t accumulate;     // y += A x instead of y = A x
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
  const __amdgpu_buffer_rsrc_t rv = buffer_of(a.val_ids ? (const void *)(a.val_ids + beg) : (const void *)(a.val + beg),
                                              (uint32_t)n * 4u);
  const __amdgpu_buffer_rsrc_t rx = buffer_of(a.x, a.xbytes);
  const __amdgpu_buffer_rsrc_t rw = buffer_of(a.val, a.val_bytes);
  const uint32_t row_bytes = (uint32_t)a.ldx * 4u, voff = (uint32_t)col0 * 4u;
  for (int32_t e0 = 0; e0 < n; e0 += G * UNROLL) {
    int32_t c[UNROLL];
    float w[UNROLL];
#pragma unroll
    for (int j = 0; j < UNROLL; ++j) {   // past the row's end: column 0, weight 0
      const int off = (e0 + j * G + g) * 4;
      c[j] = (int32_t)__builtin_amdgcn_raw_buffer_load_b32(rc, off, 0, 0);
      const unsigned v = __builtin_amdgcn_raw_buffer_load_b32(rv, off, 0, 0);
      w[j] = a.val_ids ? (e0 + j * G + g < n ? __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rw, (int)(v * 4u), 0, 0))
                                            : 0.0f)
                       : __uint_as_float(v);
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
      float4 v = make_float4(acc[0], acc[1], acc[2], acc[3]);
      if (a.accumulate) {
        const float4 o = *reinterpret_cast<const float4 *>(dst);
        v = make_float4(o.x + v.x, o.y + v.y, o.z + v.z, o.w + v.w);
      }
      *reinterpret_cast<float4 *>(dst) = v;
      return;
    }
  }
#pragma unroll
  for (int i = 0; i < V; ++i)
    if (col0 + i < a.batch) dst[i] = a.accumulate ? dst[i] + acc[i] : acc[i];
}

struct SddmmArgs {
  const int32_t *rowptr, *col;
  const float *g;         // (nrows, ldg)
  const float *x;         // (ncols, ldx)
  float *out;             // nnz, or indexed by ids
  const int32_t *ids;     // null: out[e]; else out[ids[e]] (distinct within a launch)
  int64_t ldg, ldx;
  uint32_t xbytes;
  int32_t nrows, batch, accumulate;
  uint32_t n_out;         // entries of out: ids at or past it are skipped
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
    const uint32_t slot = live ? (a.ids ? (uint32_t)a.ids[e] : (uint32_t)e) : a.n_out;
    if (slot < a.n_out) {
      float *dst = a.out + slot;
      *dst = a.accumulate ? *dst + acc : acc;
    }
  }
}

// One column (the resting trajectory's products, batch 1): 16 lanes per row or work item, four per wave.  Lane
// s of a unit takes its non-zeros s, s + 16, ..., four loads in flight per round, and the unit's 16 partial sums
// meet through xor shuffles.  A wave per row would leave most of the wave on one dependent chain of loads per
// row of ~63 non-zeros; four units per wave keep four times the loads in flight.
struct Spmv1Args {
  const int32_t *rowptr, *col;
  const float *val;
  const int32_t *val_ids;   // null, or per non-zero the index of its value in val (rows mode only)
  uint32_t val_bytes;       // bytes of val when val_ids is given (reads past it give 0)
  const float *x;           // x[col * ldx]
  float *y;                 // y[row * ldy]
  int64_t ldx, ldy;
  uint32_t xbytes;
  int32_t nrows, nnz, accumulate;
  const int4 *items;        // work items {row, first non-zero, count, slot}, or null: one unit per row
  int32_t n_items, n_slots;
  float *partials;          // slot >= 0: the unit's sum goes to partials[slot] (k_spmv_partials adds them)
};

__global__ __launch_bounds__(256) void k_spmv(const Spmv1Args a) {
  const int s = threadIdx.x & 15;
  const uint32_t unit = blockIdx.x * 16u + (threadIdx.x >> 4);
  uint32_t row = unit;
  int32_t first = 0, count = INT32_MAX, slot = -1;
  bool has = true;
  if (a.items != nullptr) {
    has = unit < (uint32_t)a.n_items;
    if (has) {
      const int4 it = a.items[unit];
      row = (uint32_t)it.x;
      first = it.y;
      count = it.z;
      slot = it.w;
      has = slot < a.n_slots;
    }
  }
  has = has && row < (uint32_t)a.nrows;
  // a malformed row pointer or work item gives wrong results, never an access outside the arrays
  int32_t beg = 0, end = 0;
  if (has) {
    const int32_t row_beg = min(max(a.rowptr[row], 0), a.nnz);
    const int32_t row_end = min(max(a.rowptr[row + 1], row_beg), a.nnz);
    beg = row_beg + min(max(first, 0), row_end - row_beg);
    end = beg + min(max(count, 0), row_end - beg);
  }
  const __amdgpu_buffer_rsrc_t rx = buffer_of(a.x, a.xbytes);
  const __amdgpu_buffer_rsrc_t rw = buffer_of(a.val, a.val_bytes);
  const uint32_t row_bytes = (uint32_t)a.ldx * 4u;
  float acc = 0.0f;
  for (int32_t e0 = beg + s; e0 < end; e0 += 64) {
    float v[4], xv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int32_t e = e0 + 16 * j;
      const bool live = e < end;
      const uint32_t c = live ? (uint32_t)a.col[e] : 0u;
      v[j] = !live ? 0.0f
             : a.val_ids ? __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rw, (int)((uint32_t)a.val_ids[e] * 4u), 0, 0))
                         : a.val[e];
      xv[j] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rx, (int)__umul24(c, row_bytes), 0, 0));
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) acc = fmaf(v[j], xv[j], acc);
  }
  acc += __shfl_xor(acc, 8);
  acc += __shfl_xor(acc, 4);
  acc += __shfl_xor(acc, 2);
  acc += __shfl_xor(acc, 1);
  if (!has || s != 0) return;
  if (slot >= 0) {
    a.partials[slot] = acc;
  } else {
    float *dst = a.y + (int64_t)row * a.ldy;
    *dst = a.accumulate ? *dst + acc : acc;
  }
}

// y[row] += the row's partial sums {row, first slot, slot count}, in slot order (one column).  The row's first
// segment wrote y[row] itself, so the sum runs first segment, then its later segments in order.
__global__ __launch_bounds__(256) void k_spmv_partials(const int4 *__restrict__ splits, int32_t n_splits,
                                                       const float *__restrict__ partials, int32_t n_slots,
                                                       float *__restrict__ y, int64_t ldy, int32_t nrows) {
  const int64_t i = blockIdx.x * 256ll + threadIdx.x;
  if (i >= n_splits) return;
  const int4 sp = splits[i];
  if ((uint32_t)sp.x >= (uint32_t)nrows || sp.y < 0 || sp.z < 0 || sp.y > n_slots - sp.z) return;
  float *dst = y + (int64_t)sp.x * ldy;
  float v = *dst;
  for (int32_t k = 0; k < sp.z; ++k) v += partials[sp.y + k];
  *dst = v;
}

// out[e] (+)= g[row_e] x[col_e] for one column: 16 lanes per row, four rows per wave, four non-zeros per lane
// in flight.  Each value is one rounded product, as k_sddmm's batch loop computes it for one column.
__global__ __launch_bounds__(256) void k_sddmm1(const SddmmArgs a) {
  const int s = threadIdx.x & 15;
  const uint32_t row = blockIdx.x * 16u + (threadIdx.x >> 4);
  if (row >= (uint32_t)a.nrows) return;
  const int32_t beg = a.rowptr[row], end = a.rowptr[row + 1];
  const float gr = a.g[(int64_t)row * a.ldg];
  const __amdgpu_buffer_rsrc_t rx = buffer_of(a.x, a.xbytes);
  const uint32_t row_bytes = (uint32_t)a.ldx * 4u;
  for (int32_t e0 = beg + s; e0 < end; e0 += 64) {
    float xv[4];
    uint32_t slot[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int32_t e = e0 + 16 * j;
      const bool live = e < end;
      xv[j] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
          rx, (int)__umul24(live ? (uint32_t)a.col[e] : 0u, row_bytes), 0, 0));
      slot[j] = live ? (a.ids ? (uint32_t)a.ids[e] : (uint32_t)e) : a.n_out;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (slot[j] < a.n_out) {
        const float v = fmaf(gr, xv[j], 0.0f);
        float *dst = a.out + slot[j];
        *dst = a.accumulate ? *dst + v : v;
      }
    }
  }
}

// ---- one recurrent step of training, elementwise parts (brain.py:313-327 under autograd) ---------------

// torch.lerp(start, end, weight) for float32 (ATen's formula: from the nearer end)
__device__ __forceinline__ float lerp_torch(float start, float end, float weight) {
  const bool small = fabsf(weight) < 0.5f;
  return fmaf(small ? weight : weight - 1.0f, end - start, small ? start : end);
}

template <int V>
struct Vec {
  float v[V];
  static __device__ __forceinline__ Vec load(const float *p) {
    Vec r;
    if constexpr (V == 4) {
      const float4 q = *reinterpret_cast<const float4 *>(p);
      r.v[0] = q.x; r.v[1] = q.y; r.v[2] = q.z; r.v[3] = q.w;
    } else {
      r.v[0] = *p;
    }
    return r;
  }
  static __device__ __forceinline__ Vec fill(float x) {
    Vec r;
#pragma unroll
    for (int i = 0; i < V; ++i) r.v[i] = x;
    return r;
  }
  __device__ __forceinline__ void store(float *p) const {
    if constexpr (V == 4)
      *reinterpret_cast<float4 *>(p) = make_float4(v[0], v[1], v[2], v[3]);
    else
      *p = v[0];
  }
};

struct StepFwdArgs {
  float *s_y;                  // in: s = A_t h_{t-1} (unless has_s == 0: s = 0); out: y, the pre-clamp drive
  int64_t lds;
  const float *k, *pdef, *a;   // per row: constant drive, resting state of the previous step, leak
  const int32_t *prev, *usrc;  // per row: row of h_{t-1} carried over (or -1), row of u (or -1); null: none
  const float *u;
  int64_t ldu;
  const float *hprev;
  int64_t ldp;
  float *h;
  int64_t ldh;
  float hmax;
  int32_t rows, batch, has_s;
};

// y = s + k + u[usrc];  x = clamp(y, 0, hmax);  p = h_{t-1}[prev] or pdef;  h = lerp(p, x, a).  One wave per
// row, V columns per lane.
template <int V>
__global__ __launch_bounds__(256) void k_train_fwd(const StepFwdArgs a) {
  const uint32_t row = blockIdx.x * 4u + (uint32_t)__builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (row >= (uint32_t)a.rows) return;
  const int lane = threadIdx.x & 63;
  const float k = a.k[row], pd = a.pdef[row], al = a.a[row];
  const int32_t pv = a.prev ? a.prev[row] : -1, us = a.usrc ? a.usrc[row] : -1;
  float *sy = a.s_y + (int64_t)row * a.lds;
  float *h = a.h + (int64_t)row * a.ldh;
  const float *ur = us >= 0 ? a.u + (int64_t)us * a.ldu : nullptr;
  const float *pr = pv >= 0 ? a.hprev + (int64_t)pv * a.ldp : nullptr;
  for (int32_t c = lane * V; c < a.batch; c += 64 * V) {
    Vec<V> s = a.has_s ? Vec<V>::load(sy + c) : Vec<V>::fill(0.0f);
    const Vec<V> u = ur ? Vec<V>::load(ur + c) : Vec<V>::fill(0.0f);
    const Vec<V> p = pr ? Vec<V>::load(pr + c) : Vec<V>::fill(pd);
    Vec<V> out;
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const float y = (s.v[i] + k) + u.v[i];
      s.v[i] = y;
      out.v[i] = lerp_torch(p.v[i], fminf(fmaxf(y, 0.0f), a.hmax), al);
    }
    s.store(sy + c);
    out.store(h + c);
  }
}

struct StepBwdArgs {
  const float *g;              // dL/dh_t
  int64_t ldg;
  const float *y;              // the forward's pre-clamp drive
  int64_t ldy;
  const float *pdef, *a;
  const int32_t *prev, *usrc;
  const float *hprev;
  int64_t ldp;
  float *gy;                   // out: dL/dy (rows, batch)
  int64_t ldgy;
  float *gk, *ga, *gpdef;      // out per row: dL/dk, dL/da, dL/dpdef
  float *gu;                   // dL/du, accumulated over steps (rows of u fed at this step are distinct)
  int64_t ldgu;
  float *ghprev;               // out: dL/dh_{t-1} of the carried rows (the caller zeroes the rest)
  int64_t ldgh;
  float hmax;
  int32_t rows, batch;
};

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

// The gradients of h = lerp(p, clamp(y, 0, hmax), a): dL/dy = g a [0 <= y <= hmax] (torch.clamp passes the
// bounds), dL/dp = g (1 - a), dL/da = sum_b g (x - p); dL/dk = sum_b dL/dy; dL/dpdef = sum_b dL/dp on rows
// that are not carried; carried rows pass dL/dp to h_{t-1}[prev]; input rows add dL/dy to u[usrc].
template <int V>
__global__ __launch_bounds__(256) void k_train_bwd(const StepBwdArgs a) {
  const uint32_t row = blockIdx.x * 4u + (uint32_t)__builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (row >= (uint32_t)a.rows) return;
  const int lane = threadIdx.x & 63;
  const float pd = a.pdef[row], al = a.a[row];
  const int32_t pv = a.prev ? a.prev[row] : -1, us = a.usrc ? a.usrc[row] : -1;
  const float *gr = a.g + (int64_t)row * a.ldg;
  const float *yr = a.y + (int64_t)row * a.ldy;
  float *gyr = a.gy + (int64_t)row * a.ldgy;
  const float *pr = pv >= 0 ? a.hprev + (int64_t)pv * a.ldp : nullptr;
  float *ghr = pv >= 0 ? a.ghprev + (int64_t)pv * a.ldgh : nullptr;
  float *gur = us >= 0 ? a.gu + (int64_t)us * a.ldgu : nullptr;
  float sk = 0.0f, sa = 0.0f, sp = 0.0f;
  for (int32_t c = lane * V; c < a.batch; c += 64 * V) {
    const Vec<V> g = Vec<V>::load(gr + c), y = Vec<V>::load(yr + c);
    const Vec<V> p = pr ? Vec<V>::load(pr + c) : Vec<V>::fill(pd);
    Vec<V> gy, gp;
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const float x = fminf(fmaxf(y.v[i], 0.0f), a.hmax);
      gy.v[i] = (y.v[i] >= 0.0f && y.v[i] <= a.hmax) ? g.v[i] * al : 0.0f;
      gp.v[i] = g.v[i] * (1.0f - al);
      sk += gy.v[i];
      sa += g.v[i] * (x - p.v[i]);
      sp += gp.v[i];
    }
    gy.store(gyr + c);
    if (ghr) gp.store(ghr + c);
    if (gur) {
      Vec<V> u = Vec<V>::load(gur + c);
#pragma unroll
      for (int i = 0; i < V; ++i) u.v[i] += gy.v[i];
      u.store(gur + c);
    }
  }
  sk = wave_sum(sk);
  sa = wave_sum(sa);
  sp = wave_sum(sp);
  if (lane == 0) {
    a.gk[row] = sk;
    a.ga[row] = sa;
    a.gpdef[row] = pv >= 0 ? 0.0f : sp;
  }
}

// ---- backward of y = A h in one pass: grad_h = A^T grad_y and dL/dw ----------------------------------
struct TransposedArgs {
  const int32_t *t_rowptr;  // CSR of A^T: rows are A's columns (rows of h)
  const int32_t *t_col;     // A's row of each non-zero (row of grad_y)
  const float *vals;        // values in A^T's order
  const int32_t *ids;       // index of each non-zero in the weight vector gw
  const float *gy;          // (rows of A, ldgy)
  const float *h;           // (rows of h, ldh)
  float *gh;                // (rows of h, ldgh)
  float *gw;                // weight gradient, += per non-zero
  int64_t ldgy, ldh, ldgh;
  uint32_t gybytes;
  int32_t nrows, batch, accumulate;
  int32_t nnz;              // non-zeros of A^T: row pointers are clamped into [0, nnz]
  uint32_t n_w;             // entries of gw: ids at or past it are skipped
  const int4 *items;        // null: one wave per row; else per wave {row, first non-zero, count, slot}
  int32_t n_items, n_slots;
  float *partials;          // (n_slots, ldgh): the state-gradient share of a row's later segments
};

// Sum over the 16 lanes of each DPP row (lanes 16 r .. 16 r + 15), in every lane of the row.
__device__ __forceinline__ float row16_sum(float v) {
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xF, 0xF, false));  // row_ror:8
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x124, 0xF, 0xF, false));  // row_ror:4
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x122, 0xF, 0xF, false));  // row_ror:2
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x121, 0xF, 0xF, false));  // row_ror:1
  return v;
}

// One wave per row j of A^T, 4 lane groups of 16 lanes x 4 columns (64 columns per chunk).  The row's
// non-zeros go in blocks of 64: group g takes non-zeros 4 r + g of the block (r = 0..15).  Per chunk every
// gathered grad_y row serves both products: it accumulates w * grad_y into grad_h[j] (the groups meet
// through the permlane sum) and its dot with h[j] accumulates into the non-zero's partial in a register, so
// dL/dw needs no second gather.  After the last chunk each group sums its 16 lanes' partials per non-zero.
//
// With a work list, a wave takes one item: a segment {first non-zero, count} of row j of A^T, longest first.
// A row's first segment (slot -1) writes grad_h[j] as above; its later segments write their share of it to
// partials[slot], which k_add_partials adds in slot order, so long rows spread over several waves and the
// sums stay deterministic.
__global__ __launch_bounds__(256) void k_transposed_backward(const TransposedArgs a) {
  constexpr int R = 16;                    // rounds per block of 64 non-zeros
  const uint32_t wave = blockIdx.x * 4u + (uint32_t)__builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  uint32_t j = wave;
  int32_t first_nz = 0, count = INT32_MAX, slot = -1;
  if (a.items != nullptr) {
    if (wave >= (uint32_t)a.n_items) return;
    const int4 it = a.items[wave];
    j = (uint32_t)it.x;
    first_nz = it.y;
    count = it.z;
    slot = it.w;
    if (slot >= a.n_slots) return;
  }
  if (j >= (uint32_t)a.nrows) return;
  const int lane = threadIdx.x & 63, g = lane >> 4, s = lane & 15;
  // a malformed row pointer or work item gives wrong results, never an access outside the arrays
  const int32_t row_beg = min(max(a.t_rowptr[j], 0), a.nnz);
  const int32_t row_end = min(max(a.t_rowptr[j + 1], row_beg), a.nnz);
  const int32_t beg = row_beg + min(max(first_nz, 0), row_end - row_beg);
  const int32_t n = min(max(count, 0), row_end - beg);
  const int32_t chunks = (a.batch + 63) / 64;
  const __amdgpu_buffer_rsrc_t rc = buffer_of(a.t_col + beg, (uint32_t)n * 4u);
  const __amdgpu_buffer_rsrc_t rv = buffer_of(a.vals + beg, (uint32_t)n * 4u);
  const __amdgpu_buffer_rsrc_t ri = buffer_of(a.ids + beg, (uint32_t)n * 4u);
  const __amdgpu_buffer_rsrc_t rgy = buffer_of(a.gy, a.gybytes);
  const uint32_t gy_row = (uint32_t)a.ldgy * 4u;
  const float *hj = a.h + (int64_t)j * a.ldh;
  float *ghj = slot < 0 ? a.gh + (int64_t)j * a.ldgh : a.partials + (int64_t)slot * a.ldgh;
  const bool add = slot < 0 && a.accumulate;   // a later segment's share starts from zero
  bool first = true;
  for (int32_t blk = 0; blk < n || (blk == 0 && !add); blk += 64) {
    // wave-uniform: the groups of 16 non-zeros wholly past the row's end are neither loaded nor gathered;
    // inside the last group the slots past the end read column 0 with weight 0 (no share of grad_h)
    const int32_t groups = min(max(n - blk, 0) + 15, R * 4) / 16;
    int32_t c[R];
    float w[R], dot[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      c[r] = 0;
      w[r] = 0.0f;
      dot[r] = 0.0f;
      if (r / 4 < groups) {
        const int off = (blk + 4 * r + g) * 4;
        c[r] = (int32_t)__builtin_amdgcn_raw_buffer_load_b32(rc, off, 0, 0);
        w[r] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rv, off, 0, 0));
      }
    }
    for (int32_t ch = 0; ch < chunks; ++ch) {
      const int32_t col0 = ch * 64 + s * 4;
      const bool live = col0 < a.batch;    // the batch is a multiple of 4 on this path
      // lanes past the batch gather zeros (an offset past any buffer of at most 2^31 - 1 bytes): their
      // columns may be a padded row's uninitialised tail, and the dot sums across the group's columns
      const uint32_t coff = live ? (uint32_t)col0 * 4u : 0x80000000u;
      float4 hv = make_float4(0.f, 0.f, 0.f, 0.f);
      if (live) hv = *reinterpret_cast<const float4 *>(hj + col0);
      float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int r0 = 0; r0 < R; r0 += 4) {
        if (r0 / 4 >= groups) break;
        float4 x[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          typedef unsigned u4 __attribute__((ext_vector_type(4)));
          const u4 v = __builtin_amdgcn_raw_buffer_load_b128(
              rgy, (int)(__umul24((uint32_t)c[r0 + q], gy_row) + coff), 0, 0);
          x[q] = make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]), __uint_as_float(v[3]));
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float wq = w[r0 + q];
          acc[0] = fmaf(wq, x[q].x, acc[0]);
          acc[1] = fmaf(wq, x[q].y, acc[1]);
          acc[2] = fmaf(wq, x[q].z, acc[2]);
          acc[3] = fmaf(wq, x[q].w, acc[3]);
          dot[r0 + q] = fmaf(x[q].x, hv.x, fmaf(x[q].y, hv.y, fmaf(x[q].z, hv.z, fmaf(x[q].w, hv.w, dot[r0 + q]))));
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] = group_sum<16>(acc[i]);
      if (g == 0 && live) {
        float4 *dst = reinterpret_cast<float4 *>(ghj + col0);
        float4 v = make_float4(acc[0], acc[1], acc[2], acc[3]);
        if (add || !first) {
          const float4 o = *dst;
          v = make_float4(o.x + v.x, o.y + v.y, o.z + v.z, o.w + v.w);
        }
        *dst = v;
      }
    }
    first = false;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (r / 4 >= groups) break;
      const float d = row16_sum(dot[r]);
      const int32_t e = blk + 4 * r + g;
      if (s == 0 && e < n) {
        const uint32_t id = __builtin_amdgcn_raw_buffer_load_b32(ri, e * 4, 0, 0);
        if (id < a.n_w) a.gw[id] += d;
      }
    }
  }
}

// The same pass in chunk-major order, for batches of more than one 64-column chunk: wave w takes chunk
// w / units of unit w % units (a work-list item, or row j without one), so the waves of one chunk run together
// and their gathers share that chunk's slice of grad_y (rows x 256 B) in L2 and the Infinity Cache instead of
// the whole of grad_y.  grad_h is written per chunk exactly as above.  Each non-zero's dot over the chunk's 64
// columns goes to dots[chunk * nnz + e] in one coalesced store per block (lane (g, s) holds the sum of round
// s), and k_dots_to_gw adds the chunks in order into gw[ids[e]].
__global__ __launch_bounds__(256) void k_transposed_backward_chunks(const TransposedArgs a, float *__restrict__ dots) {
  constexpr int R = 16;
  const uint32_t wave = blockIdx.x * 4u + (uint32_t)__builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t units = a.items != nullptr ? (uint32_t)a.n_items : (uint32_t)a.nrows;   // > 0 (host)
  const int32_t chunks = (a.batch + 63) / 64;
  const uint32_t ch = wave / units, unit = wave - ch * units;
  if (ch >= (uint32_t)chunks) return;
  uint32_t j = unit;
  int32_t first_nz = 0, count = INT32_MAX, slot = -1;
  if (a.items != nullptr) {
    const int4 it = a.items[unit];
    j = (uint32_t)it.x;
    first_nz = it.y;
    count = it.z;
    slot = it.w;
    if (slot >= a.n_slots) return;
  }
  if (j >= (uint32_t)a.nrows) return;
  const int lane = threadIdx.x & 63, g = lane >> 4, s = lane & 15;
  const int32_t row_beg = min(max(a.t_rowptr[j], 0), a.nnz);
  const int32_t row_end = min(max(a.t_rowptr[j + 1], row_beg), a.nnz);
  const int32_t beg = row_beg + min(max(first_nz, 0), row_end - row_beg);
  const int32_t n = min(max(count, 0), row_end - beg);
  const __amdgpu_buffer_rsrc_t rc = buffer_of(a.t_col + beg, (uint32_t)n * 4u);
  const __amdgpu_buffer_rsrc_t rv = buffer_of(a.vals + beg, (uint32_t)n * 4u);
  const __amdgpu_buffer_rsrc_t rgy = buffer_of(a.gy, a.gybytes);
  const uint32_t gy_row = (uint32_t)a.ldgy * 4u;
  const int32_t col0 = (int32_t)ch * 64 + s * 4;
  const bool live = col0 < a.batch;        // the batch is a multiple of 4 on this path
  // lanes past the batch gather zeros (an offset past any buffer of at most 2^31 - 1 bytes): their columns
  // may be a padded row's uninitialised tail, and the dot sums across the group's columns
  const uint32_t coff = live ? (uint32_t)col0 * 4u : 0x80000000u;
  float4 hv = make_float4(0.f, 0.f, 0.f, 0.f);
  if (live) hv = *reinterpret_cast<const float4 *>(a.h + (int64_t)j * a.ldh + col0);
  float *ghj = slot < 0 ? a.gh + (int64_t)j * a.ldgh : a.partials + (int64_t)slot * a.ldgh;
  float *drow = dots + (int64_t)ch * a.nnz + beg;   // this unit's non-zeros, [0, n), in chunk ch
  const bool add = slot < 0 && a.accumulate;
  bool first = true;
  for (int32_t blk = 0; blk < n || (blk == 0 && !add); blk += 64) {
    float dot[R], acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int r = 0; r < R; ++r) dot[r] = 0.0f;
    // Each round's records load right after the previous round's gathers: vector memory counters retire in order,
    // so the previous round's sums wait only for its gathers, and the records have those sums to arrive.
    // Wave-uniform: a group of 16 non-zeros wholly past the segment's end is not loaded; inside the last group the
    // slots past the end read column 0 with weight 0.
    auto records = [&](int r0, int32_t (&c)[4], float (&w)[4]) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int off = (blk + 4 * (r0 + q) + g) * 4;
        c[q] = (int32_t)__builtin_amdgcn_raw_buffer_load_b32(rc, off, 0, 0);
        w[q] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rv, off, 0, 0));
      }
    };
    int32_t c[4] = {0, 0, 0, 0};
    float w[4] = {0.f, 0.f, 0.f, 0.f};
    if (blk < n) records(0, c, w);
#pragma unroll
    for (int r0 = 0; r0 < R; r0 += 4) {
      if (blk + 4 * r0 >= n) break;
      float4 x[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        typedef unsigned u4 __attribute__((ext_vector_type(4)));
        const u4 v = __builtin_amdgcn_raw_buffer_load_b128(
            rgy, (int)(__umul24((uint32_t)c[q], gy_row) + coff), 0, 0);
        x[q] = make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]), __uint_as_float(v[3]));
      }
      int32_t cn[4] = {0, 0, 0, 0};
      float wn[4] = {0.f, 0.f, 0.f, 0.f};
      if (r0 + 4 < R && blk + 4 * (r0 + 4) < n) records(r0 + 4, cn, wn);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        acc[0] = fmaf(w[q], x[q].x, acc[0]);
        acc[1] = fmaf(w[q], x[q].y, acc[1]);
        acc[2] = fmaf(w[q], x[q].z, acc[2]);
        acc[3] = fmaf(w[q], x[q].w, acc[3]);
        dot[r0 + q] = fmaf(x[q].x, hv.x, fmaf(x[q].y, hv.y, fmaf(x[q].z, hv.z, x[q].w * hv.w)));
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        c[q] = cn[q];
        w[q] = wn[q];
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] = group_sum<16>(acc[i]);
    if (g == 0 && live) {
      float4 *dst = reinterpret_cast<float4 *>(ghj + col0);
      float4 v = make_float4(acc[0], acc[1], acc[2], acc[3]);
      if (add || !first) {
        const float4 o = *dst;
        v = make_float4(o.x + v.x, o.y + v.y, o.z + v.z, o.w + v.w);
      }
      *dst = v;
    }
    first = false;
    float mine = 0.0f;
#pragma unroll
    for (int r0 = 0; r0 < R; r0 += 4) {
      if (blk + 4 * r0 >= n) break;        // the same groups as above
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float d = row16_sum(dot[r0 + q]);
        mine = s == r0 + q ? d : mine;
      }
    }
    const int32_t e = blk + 4 * s + g;
    if (e < n) __builtin_nontemporal_store(mine, drow + e);
  }
}

// gw[ids[e]] += dots[0][e] + dots[1][e] + ... (chunks in order), one thread per non-zero; ids distinct, ids at or
// past n_w skipped.  With gw kept in the transposed order of the whole weight vector the ids rise with e and
// dL/dw streams.
__global__ __launch_bounds__(256) void k_dots_to_gw(const float *__restrict__ dots, int32_t nnz, int32_t chunks,
                                                    const int32_t *__restrict__ ids, uint32_t n_w,
                                                    float *__restrict__ gw) {
  const int32_t e = (int32_t)(blockIdx.x * 256u + threadIdx.x);
  if (e >= nnz) return;
  float d = dots[e];
  for (int32_t c = 1; c < chunks; ++c) d += dots[(int64_t)c * nnz + e];
  const uint32_t id = (uint32_t)ids[e];
  if (id < n_w) gw[id] += d;
}

// grad_h[row] += partials[slot_beg .. slot_beg + count) in slot order, one wave per split row
// ({row, slot_beg, count, unused} per entry); batch a multiple of 4, rows 16-byte aligned.
__global__ __launch_bounds__(256) void k_add_partials(const int4 *__restrict__ splits, int32_t n_splits,
                                                      const float *__restrict__ partials, int32_t n_slots,
                                                      float *__restrict__ gh, int64_t ldgh, int32_t nrows,
                                                      int32_t batch) {
  const uint32_t w = blockIdx.x * 4u + (uint32_t)__builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (w >= (uint32_t)n_splits) return;
  const int4 sp = splits[w];
  if ((uint32_t)sp.x >= (uint32_t)nrows || sp.y < 0 || sp.z < 0 || sp.y > n_slots - sp.z) return;
  float *dst = gh + (int64_t)sp.x * ldgh;
  for (int32_t c = (threadIdx.x & 63) * 4; c < batch; c += 256) {
    float4 v = *reinterpret_cast<const float4 *>(dst + c);
    for (int32_t k = 0; k < sp.z; ++k) {
      const float4 p = *reinterpret_cast<const float4 *>(partials + (int64_t)(sp.y + k) * ldgh + c);
      v = make_float4(v.x + p.x, v.y + p.y, v.z + p.z, v.w + p.w);
    }
    *reinterpret_cast<float4 *>(dst + c) = v;
  }
}

// ---- the resting trajectory under training (brain.py:238-252, one column) ----------------------------
// c_t = lerp(c_{t-1}, clamp(W c_{t-1} + b, 0, H), alpha) over the whole network, and the drive the rows of R_t
// get from outside the light cone, k_t = (W c_{t-1} + b - A_t c_{t-1}[R_{t-1}])[R_t], which is the same sum
// over the edges whose presynaptic neuron lies outside R_{t-1}.  One pass over W gathers, per edge, the pair
// x2[j] = {c_{t-1}[j], c_{t-1}[j] if j is outside R_{t-1} else 0} and keeps both sums; the full one is summed
// in k_spmv's order, so c_t has the same bits as a separate product would give.

struct RestFwdArgs {
  const int32_t *crow, *pre;   // W in CSR, rows = postsynaptic neurons
  const float *w;
  const float2 *x2;            // the pairs of c_{t-1}, or null: c_{t-1} = 0 and no edge terms
  const float *bias, *alpha;   // alpha: sigmoid(alpha_logit), n
  const float *c_prev;         // c_{t-1}, or null: 0
  const uint8_t *member;       // neurons of R_t, or null: none (builds the next step's pairs)
  float *full, *outside, *c_next;
  float2 *x2_next;
  float hmax;
  int32_t n, nnz;
  uint32_t x2bytes;
};

__global__ __launch_bounds__(256) void k_rest_fwd(const RestFwdArgs a) {
  const int s = threadIdx.x & 15;
  const uint32_t row = blockIdx.x * 16u + (threadIdx.x >> 4);
  const bool has = row < (uint32_t)a.n;
  float acc = 0.0f, out = 0.0f;
  if (has && a.x2 != nullptr) {
    const int32_t beg = min(max(a.crow[row], 0), a.nnz);
    const int32_t end = min(max(a.crow[row + 1], beg), a.nnz);
    const __amdgpu_buffer_rsrc_t rx = buffer_of(a.x2, a.x2bytes);
    for (int32_t e0 = beg + s; e0 < end; e0 += 64) {
      float v[4];
      float2 xv[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int32_t e = e0 + 16 * j;
        const bool live = e < end;
        v[j] = live ? a.w[e] : 0.0f;
        xv[j] = __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(
                                               rx, (int)((live ? (uint32_t)a.pre[e] : 0u) * 8u), 0, 0));
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        acc = fmaf(v[j], xv[j].x, acc);
        out = fmaf(v[j], xv[j].y, out);
      }
    }
  }
#pragma unroll
  for (int off = 8; off > 0; off >>= 1) {
    acc += __shfl_xor(acc, off);
    out += __shfl_xor(out, off);
  }
  if (!has || s != 0) return;
  const float b = a.bias[row];
  const float f = acc + b;
  a.full[row] = f;
  a.outside[row] = out + b;
  const float cn = lerp_torch(a.c_prev ? a.c_prev[row] : 0.0f, fminf(fmaxf(f, 0.0f), a.hmax), a.alpha[row]);
  a.c_next[row] = cn;
  a.x2_next[row] = make_float2(cn, (a.member && a.member[row]) ? 0.0f : cn);
}

// The backward of one step's elementwise part (torch.lerp's and clamp's gradients), per neuron: from
// dL/dc_t, dL/dk_t and dL/dp_t (p_t = c_{t-1}[R_t], both scattered through pos = each neuron's place in R_t
// or -1), the pair g2 = {dL/dfull, dL/doutside} for the products, dL/dc_{t-1} through the lerp and p_t, and
// the bias and alpha gradients (accumulated).
struct RestBwdArgs {
  const float *gc;             // dL/dc_t, or null: 0
  const int32_t *pos;
  const float *gk, *gp;        // |R_t| each, or null: 0
  const float *full, *c_prev, *alpha;   // c_prev null: 0
  float2 *g2;
  float *gc_prev, *gbias, *galpha;
  float hmax;
  int32_t n;
};

__global__ __launch_bounds__(256) void k_rest_bwd(const RestBwdArgs a) {
  const int64_t i = blockIdx.x * 256ll + threadIdx.x;
  if (i >= a.n) return;
  const float g = a.gc ? a.gc[i] : 0.0f;
  const float al = a.alpha[i], f = a.full[i];
  const float cp = a.c_prev ? a.c_prev[i] : 0.0f;
  const int32_t p = a.pos[i];
  const float gout = (p >= 0 && a.gk) ? a.gk[p] : 0.0f;
  const float gfull = (f >= 0.0f && f <= a.hmax) ? g * al : 0.0f;   // clamp passes its bounds
  a.g2[i] = make_float2(gfull, gout);
  a.gbias[i] += gfull + gout;
  a.galpha[i] += g * (fminf(fmaxf(f, 0.0f), a.hmax) - cp);
  a.gc_prev[i] = g * (1.0f - al) + ((p >= 0 && a.gp) ? a.gp[p] : 0.0f);
}

// dL/dw_e += g2[post_e] . x2[pre_e] over W's rows (16 lanes per row): the full product's and the outside
// sum's shares of each weight gradient in one pass.
__global__ __launch_bounds__(256) void k_rest_sddmm(const int32_t *__restrict__ crow, const int32_t *__restrict__ pre,
                                                    int32_t n, int32_t nnz, const float2 *__restrict__ g2,
                                                    const float2 *__restrict__ x2, uint32_t x2bytes,
                                                    float *__restrict__ gw) {
  const int s = threadIdx.x & 15;
  const uint32_t row = blockIdx.x * 16u + (threadIdx.x >> 4);
  if (row >= (uint32_t)n) return;
  const float2 gr = g2[row];
  if (gr.x == 0.0f && gr.y == 0.0f) return;          // adds of 0 change nothing
  const int32_t beg = min(max(crow[row], 0), nnz), end = min(max(crow[row + 1], beg), nnz);
  const __amdgpu_buffer_rsrc_t rx = buffer_of(x2, x2bytes);
  for (int32_t e0 = beg + s; e0 < end; e0 += 64) {
    float2 xv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int32_t e = e0 + 16 * j;
      xv[j] = __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(
                                             rx, (int)((e < end ? (uint32_t)pre[e] : 0u) * 8u), 0, 0));
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int32_t e = e0 + 16 * j;
      if (e < end) gw[e] += fmaf(gr.x, xv[j].x, gr.y * xv[j].y);
    }
  }
}

// dL/dc_{t-1}[j] += sum over W^T's row j of w_e (g2[post_e].x + (j outside R_{t-1} ? g2[post_e].y : 0)), over
// the work list of W^T (as k_spmv's work items: first segments write, later ones go to partial slots).
struct RestTArgs {
  const int32_t *rowptr, *col;
  const float *val;
  const float2 *g2;
  uint32_t g2bytes;
  const uint8_t *member_prev;  // neurons of R_{t-1}, or null: none
  float *y;
  int32_t nrows, nnz;
  const int4 *items;
  int32_t n_items, n_slots;
  float *partials;
};

__global__ __launch_bounds__(256) void k_rest_spmv_t(const RestTArgs a) {
  const int s = threadIdx.x & 15;
  const uint32_t unit = blockIdx.x * 16u + (threadIdx.x >> 4);
  bool has = unit < (uint32_t)a.n_items;
  uint32_t row = 0;
  int32_t beg = 0, end = 0, slot = -1;
  if (has) {
    const int4 it = a.items[unit];
    row = (uint32_t)it.x;
    slot = it.w;
    has = row < (uint32_t)a.nrows && slot < a.n_slots;
    if (has) {
      const int32_t row_beg = min(max(a.rowptr[row], 0), a.nnz);
      const int32_t row_end = min(max(a.rowptr[row + 1], row_beg), a.nnz);
      beg = row_beg + min(max(it.y, 0), row_end - row_beg);
      end = beg + min(max(it.z, 0), row_end - beg);
    }
  }
  const bool outside = has && !(a.member_prev && a.member_prev[row]);
  const __amdgpu_buffer_rsrc_t rx = buffer_of(a.g2, a.g2bytes);
  float acc = 0.0f;
  for (int32_t e0 = beg + s; e0 < end; e0 += 64) {
    float v[4];
    float2 xv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int32_t e = e0 + 16 * j;
      const bool live = e < end;
      v[j] = live ? a.val[e] : 0.0f;
      xv[j] = __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(
                                             rx, (int)((live ? (uint32_t)a.col[e] : 0u) * 8u), 0, 0));
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) acc = fmaf(v[j], outside ? xv[j].x + xv[j].y : xv[j].x, acc);
  }
#pragma unroll
  for (int off = 8; off > 0; off >>= 1) acc += __shfl_xor(acc, off);
  if (!has || s != 0) return;
  if (slot >= 0)
    a.partials[slot] = acc;
  else
    a.y[row] += acc;
}

// out[i] = w[ids[i]]: a sub-matrix's weights in its own (or its transpose's) order, from int32 ids in one pass;
// ids past the weight vector read 0.
__global__ __launch_bounds__(256) void k_gather_values(const float *__restrict__ w, uint32_t wbytes,
                                                       const int32_t *__restrict__ ids, int64_t n,
                                                       float *__restrict__ out) {
  const __amdgpu_buffer_rsrc_t rw = buffer_of(w, wbytes);
  for (int64_t i = blockIdx.x * 256ll + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const uint32_t id = (uint32_t)ids[i];
    out[i] = id < wbytes / 4u ? __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rw, (int)(id * 4u), 0, 0)) : 0.0f;
  }
}

// records[i] = {col[i], the bits of w[ids[i]]} (w[i] without ids; ids past n_w give 0): a structure's {column,
// value} records for the swept products in one pass, from the columns and the whole weight vector
__global__ __launch_bounds__(256) void k_gather_records(const int32_t *__restrict__ col, const float *__restrict__ w,
                                                        uint32_t wbytes, const int32_t *__restrict__ ids, int64_t n,
                                                        int2 *__restrict__ records) {
  const __amdgpu_buffer_rsrc_t rw = buffer_of(w, wbytes);
  for (int64_t i = blockIdx.x * 256ll + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const uint32_t id = ids ? (uint32_t)ids[i] : (uint32_t)i;
    const uint32_t v = id < wbytes / 4u ? __builtin_amdgcn_raw_buffer_load_b32(rw, (int)(id * 4u), 0, 0) : 0u;
    records[i] = make_int2(col[i], (int)v);
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

extern "C" size_t fly_spmm_swept_workspace(const fly_sweep *sweep, int64_t batch) {
  return sweep ? sweep_pieces_bytes(sweep->t.get(), batch) : 0;
}

extern "C" int fly_spmm_swept(const fly_sweep *sweep, const void *records, int64_t nnz, const float *x, int64_t ldx,
                              int64_t batch, float *y, int64_t ldy, void *ws, size_t ws_bytes, void *stream) {
  return guard([&] {
    FLY_REQUIRE(sweep && sweep->t && records && x && y, "null argument");
    FLY_REQUIRE(current_device() == sweep->device, "the sweep tables live on another device");
    const SweepTables &t = *sweep->t;
    // the tables index the records: they must be the structure's nnz records, in its CSR order
    FLY_REQUIRE(nnz == t.nnz, "the records do not match the structure's non-zeros");
    FLY_REQUIRE(batch > 0 && batch % 4 == 0 && batch < (int64_t)INT32_MAX / 2, "the batch must be a multiple of 4");
    FLY_REQUIRE(ldx >= batch && ldy >= batch && ldx % 4 == 0 && ldy % 4 == 0 && aligned(x, 16) && aligned(y, 16),
                "x and y rows must be 16-byte aligned and hold the batch");
    const size_t need = sweep_pieces_bytes(&t, batch);
    FLY_REQUIRE(need == 0 || (ws && ws_bytes >= need && aligned(ws, 256)), "workspace too small or misaligned");
    const uint32_t xbytes = buffer_bytes(t.ncols, ldx, sizeof(float));
    FLY_REQUIRE(xbytes != 0, "x must be below 2 GiB with rows of 24-bit indices");
    StepArgs<float, float> a{};
    a.colval = static_cast<const int2 *>(records);
    a.xprev = x;
    a.ldx = ldx;
    a.xout = y;
    a.ldo = ldy;
    a.nrows = (int32_t)t.nrows;
    a.batch = (int32_t)batch;
    a.xbytes = xbytes;
    a.pieces = static_cast<float *>(ws);
    a.sweep_paired = sweep->tune.sweep_paired;
    a.sweep_slots = sweep->tune.sweep_slots;
    a.sweep_pipe = sweep->tune.sweep_pipe;
    a.sweep_exact = 1;   // x is the caller's: it may hold inf or NaN
    LaunchTimer timer(FLY_K_OTHER, as_stream(stream));
    launch_swept<float, float, 3>(a, t, as_stream(stream));
    check_launch("swept product");
  });
}

namespace {
// dL/dw's dots of a swept transposed backward: one float per record and chunk of 32 columns, after the pieces' sums
size_t swept_backward_dots_bytes(const SweepTables &t, int64_t batch) {
  return (size_t)((batch + 31) / 32) * (size_t)t.nnz * sizeof(float);
}
}  // namespace

extern "C" size_t fly_transposed_backward_swept_workspace(const fly_sweep *sweep, int64_t batch) {
  if (!sweep || !sweep->t || batch <= 0) return 0;
  return align256(sweep_pieces_bytes(sweep->t.get(), batch)) + swept_backward_dots_bytes(*sweep->t, batch);
}

extern "C" int fly_transposed_backward_swept(const fly_sweep *sweep, const void *records, int64_t nnz,
                                             const int32_t *ids, const float *gy, int64_t ldgy, const float *h,
                                             int64_t ldh, int64_t batch, float *gh, int64_t ldgh, int32_t accumulate,
                                             float *gw, int64_t n_w, void *ws, size_t ws_bytes, void *stream) {
  return guard([&] {
    FLY_REQUIRE(sweep && sweep->t && records && ids && gy && h && gh && gw, "null argument");
    FLY_REQUIRE(current_device() == sweep->device, "the sweep tables live on another device");
    const SweepTables &t = *sweep->t;
    // the tables index the records: they must be the structure's nnz records, in its CSR order
    FLY_REQUIRE(nnz == t.nnz, "the records do not match the structure's non-zeros");
    FLY_REQUIRE(batch > 0 && batch % 4 == 0 && batch < (int64_t)INT32_MAX / 2, "the batch must be a multiple of 4");
    FLY_REQUIRE(vec4_ok(gy, ldgy) && vec4_ok(h, ldh) && vec4_ok(gh, ldgh) && ldgy >= batch && ldh >= batch &&
                    ldgh >= batch,
                "gy, h and gh rows must be 16-byte aligned and hold the batch");
    FLY_REQUIRE(n_w >= 0 && n_w < (int64_t)1 << 32, "n_w out of range");
    const size_t pieces = align256(sweep_pieces_bytes(&t, batch));
    FLY_REQUIRE(ws && aligned(ws, 256) && ws_bytes >= pieces + swept_backward_dots_bytes(t, batch),
                "workspace too small or misaligned");
    const uint32_t xbytes = buffer_bytes(t.ncols, ldgy, sizeof(float));
    FLY_REQUIRE(xbytes != 0, "gy must be below 2 GiB with rows of 24-bit indices");
    StepArgs<float, float> a{};
    a.colval = static_cast<const int2 *>(records);
    a.xprev = gy;
    a.ldx = ldgy;
    a.xout = gh;
    a.ldo = ldgh;
    a.nrows = (int32_t)t.nrows;
    a.batch = (int32_t)batch;
    a.xbytes = xbytes;
    a.pieces = static_cast<float *>(ws);
    a.hdot = h;
    a.ldh = ldh;
    a.dots = reinterpret_cast<float *>(static_cast<char *>(ws) + pieces);
    a.ndots = nnz;
    a.piece_row = t.piece_row.p;
    a.accumulate = accumulate != 0;
    LaunchTimer timer(FLY_K_OTHER, as_stream(stream));
    launch_swept<float, float, 4>(a, t, as_stream(stream));
    check_launch("swept transposed backward");
    hipLaunchKernelGGL(k_dots_to_gw, dim3(blocks_for(nnz, 256)), dim3(256), 0, as_stream(stream), a.dots,
                       (int32_t)nnz, (int32_t)((batch + 31) / 32), ids, (uint32_t)n_w, gw);
    check_launch("dots to gw");
  });
}

extern "C" int fly_spmm(const int32_t *rowptr, const int32_t *col, const float *val, const int32_t *val_ids,
                        int64_t n_val, int64_t nrows, int64_t ncols, const float *x, int64_t ldx, int64_t batch,
                        float *y, int64_t ldy, int32_t accumulate, void *stream) {
  return guard([&] {
    FLY_REQUIRE(nrows >= 0 && ncols >= 0 && batch >= 0, "negative size");
    FLY_REQUIRE(nrows < (int64_t)1 << 24 && ncols < (int64_t)1 << 24, "more than 2^24 rows or columns");
    if (!nrows || !batch) return;
    FLY_REQUIRE(rowptr && y && ldy >= batch, "bad argument");
    FLY_REQUIRE(ncols == 0 || (col && val && x && ldx >= batch && ldx < (1 << 22)), "bad argument");
    LaunchTimer timer(FLY_K_OTHER, as_stream(stream));
    FLY_REQUIRE(!val_ids || (n_val >= 0 && n_val < (int64_t)1 << 29), "n_val out of range");
    SpmmArgs a{rowptr, col, val, val_ids, (uint32_t)(val_ids ? n_val * 4 : 0), x, y, ldx, ldy,
               checked_bytes(ncols, ldx), (int32_t)nrows, (int32_t)batch, 0, accumulate != 0};
    if (ncols == 0) a.xbytes = 0;   // every gather reads zeros: y = 0
    // one column: lanes across the non-zeros; else 16-byte lanes in groups of 16 (64 columns per chunk) when
    // the rows allow them, else 4-byte lanes in groups of 8
    if (batch == 1) {
      Spmv1Args b{rowptr, col, val, val_ids, a.val_bytes, x, y, ldx, ldy, a.xbytes, (int32_t)nrows, INT32_MAX,
                  accumulate != 0, nullptr, 0, 0, nullptr};
      hipLaunchKernelGGL(k_spmv, dim3(blocks_for(nrows, 16)), dim3(256), 0, as_stream(stream), b);
    } else if (batch >= 4 && vec4_ok(x, ldx) && vec4_ok(y, ldy)) {
      const int tg = tuning_snapshot().spmm_groups;
      const int g = tg == 2 || tg == 8 ? tg : 4;
      const int width = 64 / g * 4;   // columns per chunk
      a.chunks = (int32_t)((batch + width - 1) / width);
      if (g == 2)
        launch_spmm<2, 4>(a, as_stream(stream));
      else if (g == 8)
        launch_spmm<8, 4>(a, as_stream(stream));
      else
        launch_spmm<4, 4>(a, as_stream(stream));
    } else {
      a.chunks = (int32_t)((batch + 7) / 8);
      launch_spmm<8, 1>(a, as_stream(stream));
    }
    check_launch("spmm");
  });
}

extern "C" int fly_sddmm(const int32_t *rowptr, const int32_t *col, int64_t nrows, int64_t ncols, const float *g,
                         int64_t ldg, const float *x, int64_t ldx, int64_t batch, float *out, int64_t n_out,
                         const int32_t *ids, int32_t accumulate, void *stream) {
  return guard([&] {
    FLY_REQUIRE(nrows >= 0 && ncols >= 0 && batch >= 0, "negative size");
    FLY_REQUIRE(nrows < (int64_t)1 << 24 && ncols < (int64_t)1 << 24, "more than 2^24 rows or columns");
    if (!nrows) return;
    FLY_REQUIRE(rowptr && col && out && g && ldg >= batch, "bad argument");
    FLY_REQUIRE(ncols == 0 || (x && ldx >= batch && ldx < (1 << 22)), "bad argument");
    LaunchTimer timer(FLY_K_OTHER, as_stream(stream));
    FLY_REQUIRE(n_out >= 0 && n_out < (int64_t)1 << 32, "n_out out of range");
    SddmmArgs a{rowptr, col, g, x, out, ids, ldg, ldx, ncols ? checked_bytes(ncols, ldx) : 0u, (int32_t)nrows,
                (int32_t)batch, accumulate != 0, (uint32_t)n_out};
    const dim3 grid(blocks_for(nrows, 4)), block(256);
    if (batch == 1)
      hipLaunchKernelGGL(k_sddmm1, dim3(blocks_for(nrows, 16)), block, 0, as_stream(stream), a);
    else if (batch >= 4 && vec4_ok(x, ldx))
      hipLaunchKernelGGL(k_sddmm<4>, grid, block, 0, as_stream(stream), a);
    else
      hipLaunchKernelGGL(k_sddmm<1>, grid, block, 0, as_stream(stream), a);
    check_launch("sddmm");
  });
}

extern "C" int fly_spmv_work(const int32_t *rowptr, const int32_t *col, const float *val, int64_t nnz, int64_t nrows,
                             int64_t ncols, const float *x, int64_t ldx, float *y, int64_t ldy, int32_t accumulate,
                             const int32_t *items, int64_t n_items, const int32_t *splits, int64_t n_splits,
                             float *partials, int64_t n_slots, void *stream) {
  return guard([&] {
    FLY_REQUIRE(nrows >= 0 && ncols >= 0 && nnz >= 0 && n_items >= 0 && n_splits >= 0 && n_slots >= 0, "negative size");
    FLY_REQUIRE(nrows < (int64_t)1 << 24 && ncols < (int64_t)1 << 24, "more than 2^24 rows or columns");
    FLY_REQUIRE(nnz < (int64_t)INT32_MAX && n_items < (int64_t)INT32_MAX && n_splits < (int64_t)INT32_MAX &&
                n_slots < (int64_t)INT32_MAX, "size out of range");
    if (!nrows || !n_items) return;
    FLY_REQUIRE(rowptr && y && ldy >= 1 && items, "bad argument");
    FLY_REQUIRE(nnz == 0 || (col && val), "bad argument");
    FLY_REQUIRE(ncols == 0 || (x && ldx >= 1 && ldx < (1 << 22)), "bad argument");
    FLY_REQUIRE((n_splits == 0 || splits) && (n_slots == 0 || partials), "split rows need splits and partials");
    LaunchTimer timer(FLY_K_OTHER, as_stream(stream));
    Spmv1Args a{rowptr, col, val, nullptr, 0u, x, y, ldx, ldy, ncols ? checked_bytes(ncols, ldx) : 0u,
                (int32_t)nrows, (int32_t)nnz, accumulate != 0, reinterpret_cast<const int4 *>(items),
                (int32_t)n_items, (int32_t)n_slots, partials};
    hipLaunchKernelGGL(k_spmv, dim3(blocks_for(n_items, 16)), dim3(256), 0, as_stream(stream), a);
    if (n_splits)
      hipLaunchKernelGGL(k_spmv_partials, dim3(blocks_for(n_splits, 256)), dim3(256), 0, as_stream(stream),
                         reinterpret_cast<const int4 *>(splits), (int32_t)n_splits, partials, (int32_t)n_slots, y, ldy,
                         (int32_t)nrows);
    check_launch("spmv work");
  });
}

extern "C" int fly_rest_forward(const int32_t *crow, const int32_t *pre, const float *w, int64_t n, int64_t nnz,
                                const float *x2, const float *bias, const float *alpha, const float *c_prev,
                                float h_max, const uint8_t *member, float *full, float *outside, float *c_next,
                                float *x2_next, void *stream) {
  return guard([&] {
    FLY_REQUIRE(n >= 0 && n < (int64_t)1 << 28 && nnz >= 0 && nnz < (int64_t)INT32_MAX, "size out of range");
    if (!n) return;
    FLY_REQUIRE(crow && bias && alpha && full && outside && c_next && x2_next, "bad argument");
    FLY_REQUIRE(!x2 || (nnz == 0 || (pre && w)), "bad argument");
    LaunchTimer timer(FLY_K_OTHER, as_stream(stream));
    RestFwdArgs a{crow, pre, w, reinterpret_cast<const float2 *>(x2), bias, alpha, c_prev, member, full, outside,
                  c_next, reinterpret_cast<float2 *>(x2_next), h_max, (int32_t)n, (int32_t)nnz,
                  (uint32_t)(n * 8)};
    hipLaunchKernelGGL(k_rest_fwd, dim3(blocks_for(n, 16)), dim3(256), 0, as_stream(stream), a);
    check_launch("resting step");
  });
}

extern "C" int fly_rest_backward(const float *gc, const int32_t *pos, const float *gk, const float *gp,
                                 const float *full, const float *c_prev, const float *alpha, float h_max, int64_t n,
                                 float *g2, float *gc_prev, float *gbias, float *galpha, void *stream) {
  return guard([&] {
    FLY_REQUIRE(n >= 0 && n < (int64_t)1 << 28, "size out of range");
    if (!n) return;
    FLY_REQUIRE(pos && full && alpha && g2 && gc_prev && gbias && galpha, "bad argument");
    LaunchTimer timer(FLY_K_OTHER, as_stream(stream));
    RestBwdArgs a{gc, pos, gk, gp, full, c_prev, alpha, reinterpret_cast<float2 *>(g2), gc_prev, gbias, galpha,
                  h_max, (int32_t)n};
    hipLaunchKernelGGL(k_rest_bwd, dim3(blocks_for(n, 256)), dim3(256), 0, as_stream(stream), a);
    check_launch("resting step backward");
  });
}

extern "C" int fly_rest_products_backward(const int32_t *crow, const int32_t *pre, int64_t n, int64_t nnz,
                                          const float *g2, const float *x2, float *gw, const int32_t *t_rowptr,
                                          const int32_t *t_col, const float *t_val, const uint8_t *member_prev,
                                          const int32_t *items, int64_t n_items, const int32_t *splits,
                                          int64_t n_splits, float *partials, int64_t n_slots, float *gc_prev,
                                          void *stream) {
  return guard([&] {
    FLY_REQUIRE(n >= 0 && n < (int64_t)1 << 28 && nnz >= 0 && nnz < (int64_t)INT32_MAX, "size out of range");
    FLY_REQUIRE(n_items >= 0 && n_items < (int64_t)INT32_MAX && n_splits >= 0 && n_splits < (int64_t)INT32_MAX &&
                n_slots >= 0 && n_slots < (int64_t)INT32_MAX, "work list out of range");
    if (!n) return;
    FLY_REQUIRE(crow && g2 && x2 && gw && t_rowptr && gc_prev && (n_items == 0 || items), "bad argument");
    FLY_REQUIRE(nnz == 0 || (pre && t_col && t_val), "bad argument");
    FLY_REQUIRE((n_splits == 0 || splits) && (n_slots == 0 || partials), "split rows need splits and partials");
    LaunchTimer timer(FLY_K_OTHER, as_stream(stream));
    hipStream_t st = as_stream(stream);
    const uint32_t pair_bytes = (uint32_t)(n * 8);
    hipLaunchKernelGGL(k_rest_sddmm, dim3(blocks_for(n, 16)), dim3(256), 0, st, crow, pre, (int32_t)n, (int32_t)nnz,
                       reinterpret_cast<const float2 *>(g2), reinterpret_cast<const float2 *>(x2), pair_bytes, gw);
    if (n_items) {
      RestTArgs a{t_rowptr, t_col, t_val, reinterpret_cast<const float2 *>(g2), pair_bytes, member_prev, gc_prev,
                  (int32_t)n, (int32_t)nnz, reinterpret_cast<const int4 *>(items), (int32_t)n_items,
                  (int32_t)n_slots, partials};
      hipLaunchKernelGGL(k_rest_spmv_t, dim3(blocks_for(n_items, 16)), dim3(256), 0, st, a);
      if (n_splits)
        hipLaunchKernelGGL(k_spmv_partials, dim3(blocks_for(n_splits, 256)), dim3(256), 0, st,
                           reinterpret_cast<const int4 *>(splits), (int32_t)n_splits, partials, (int32_t)n_slots,
                           gc_prev, (int64_t)1, (int32_t)n);
    }
    check_launch("resting products backward");
  });
}

extern "C" int fly_gather_values(const float *w, int64_t n_w, const int32_t *ids, int64_t n, float *out,
                                 void *stream) {
  return guard([&] {
    FLY_REQUIRE(n_w >= 0 && n_w < (int64_t)1 << 29 && n >= 0 && n < (int64_t)1 << 40, "size out of range");
    if (!n) return;
    FLY_REQUIRE(ids && out && (n_w == 0 || w), "bad argument");
    LaunchTimer timer(FLY_K_OTHER, as_stream(stream));
    const int64_t blocks = std::min<int64_t>(blocks_for(n, 256), 65536);
    hipLaunchKernelGGL(k_gather_values, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream), w,
                       (uint32_t)(n_w * 4), ids, n, out);
    check_launch("gather values");
  });
}

namespace {
// float64 products for modules converted to float64 (the reference's .double() tests): plain and exact, one wave per
// row with the lanes over the batch columns, each sum in CSR order.  Row pointers are clamped into [0, nnz], values
// read at e or val_ids[e] only below n_val and columns only below ncols, so a malformed structure gives wrong
// results, never an access outside the arrays.
__global__ __launch_bounds__(256) void k_spmm_f64(const int32_t *__restrict__ rowptr, const int32_t *__restrict__ col,
                                                  int64_t nnz, const double *__restrict__ val,
                                                  const int32_t *__restrict__ val_ids, int64_t n_val, int64_t nrows,
                                                  int64_t ncols, const double *__restrict__ x, int64_t ldx,
                                                  int64_t batch, double *__restrict__ y, int64_t ldy, int accumulate) {
  const int64_t r = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= nrows) return;
  const int lane = threadIdx.x & 63;
  const int64_t beg = min(max((int64_t)rowptr[r], (int64_t)0), nnz);
  const int64_t end = min(max((int64_t)rowptr[r + 1], beg), nnz);
  for (int64_t b = lane; b < batch; b += 64) {
    double acc = 0.0;
    for (int64_t e = beg; e < end; ++e) {
      const int64_t v = val_ids ? (int64_t)val_ids[e] : e;
      const int64_t c = col[e];
      if (v >= 0 && v < n_val && c >= 0 && c < ncols) acc = fma(val[v], x[c * ldx + b], acc);
    }
    double *dst = y + r * ldy + b;
    *dst = accumulate ? *dst + acc : acc;
  }
}

// out[ids ? ids[e] : e] (+)= sum_b g[row_e, b] x[col_e, b]: one wave per row, a lane per non-zero (ids distinct; ids
// at or past n_out skipped)
__global__ __launch_bounds__(256) void k_sddmm_f64(const int32_t *__restrict__ rowptr, const int32_t *__restrict__ col,
                                                   int64_t nnz, int64_t nrows, int64_t ncols,
                                                   const double *__restrict__ g, int64_t ldg,
                                                   const double *__restrict__ x, int64_t ldx, int64_t batch,
                                                   double *__restrict__ out, int64_t n_out,
                                                   const int32_t *__restrict__ ids, int accumulate) {
  const int64_t r = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= nrows) return;
  const int lane = threadIdx.x & 63;
  const int64_t beg = min(max((int64_t)rowptr[r], (int64_t)0), nnz);
  const int64_t end = min(max((int64_t)rowptr[r + 1], beg), nnz);
  for (int64_t e = beg + lane; e < end; e += 64) {
    const int64_t c = col[e];
    const int64_t slot = ids ? (int64_t)ids[e] : e;
    if (c < 0 || c >= ncols || slot < 0 || slot >= n_out) continue;
    double acc = 0.0;
    for (int64_t b = 0; b < batch; ++b) acc = fma(g[r * ldg + b], x[c * ldx + b], acc);
    out[slot] = accumulate ? out[slot] + acc : acc;
  }
}
}  // namespace

extern "C" int fly_spmm_f64(const int32_t *rowptr, const int32_t *col, int64_t nnz, const double *val,
                            const int32_t *val_ids, int64_t n_val, int64_t nrows, int64_t ncols, const double *x,
                            int64_t ldx, int64_t batch, double *y, int64_t ldy, int32_t accumulate, void *stream) {
  return guard([&] {
    FLY_REQUIRE(nrows >= 0 && ncols >= 0 && batch >= 0 && nnz >= 0 && n_val >= 0, "negative size");
    if (!nrows || !batch) return;
    FLY_REQUIRE(rowptr && y && ldy >= batch, "bad argument");
    FLY_REQUIRE(nnz == 0 || (col && val && x && ldx >= batch), "bad argument");
    LaunchTimer timer(FLY_K_OTHER, as_stream(stream));
    hipLaunchKernelGGL(k_spmm_f64, dim3(blocks_for(nrows, 4)), dim3(256), 0, as_stream(stream), rowptr, col, nnz, val,
                       val_ids, n_val, nrows, ncols, x, ldx, batch, y, ldy, (int)(accumulate != 0));
    check_launch("spmm f64");
  });
}

extern "C" int fly_sddmm_f64(const int32_t *rowptr, const int32_t *col, int64_t nnz, int64_t nrows, int64_t ncols,
                             const double *g, int64_t ldg, const double *x, int64_t ldx, int64_t batch, double *out,
                             int64_t n_out, const int32_t *ids, int32_t accumulate, void *stream) {
  return guard([&] {
    FLY_REQUIRE(nrows >= 0 && ncols >= 0 && batch >= 0 && nnz >= 0 && n_out >= 0, "negative size");
    if (!nrows || !nnz) return;
    FLY_REQUIRE(rowptr && col && out && (batch == 0 || (g && x && ldg >= batch && ldx >= batch)), "bad argument");
    LaunchTimer timer(FLY_K_OTHER, as_stream(stream));
    hipLaunchKernelGGL(k_sddmm_f64, dim3(blocks_for(nrows, 4)), dim3(256), 0, as_stream(stream), rowptr, col, nnz,
                       nrows, ncols, g, ldg, x, ldx, batch, out, n_out, ids, (int)(accumulate != 0));
    check_launch("sddmm f64");
  });
}

extern "C" int fly_gather_records(const int32_t *col, const float *w, int64_t n_w, const int32_t *ids, int64_t n,
                                  void *records, void *stream) {
  return guard([&] {
    FLY_REQUIRE(n_w >= 0 && n_w < (int64_t)1 << 29 && n >= 0 && n < (int64_t)1 << 40, "size out of range");
    if (!n) return;
    FLY_REQUIRE(col && records && aligned(records, 8) && (n_w == 0 || w), "bad argument");
    LaunchTimer timer(FLY_K_OTHER, as_stream(stream));
    const int64_t blocks = std::min<int64_t>(blocks_for(n, 256), 65536);
    hipLaunchKernelGGL(k_gather_records, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream), col, w,
                       (uint32_t)(n_w * 4), ids, n, static_cast<int2 *>(records));
    check_launch("gather records");
  });
}

extern "C" int fly_train_step_forward(int64_t rows, int64_t batch, float *s_y, int64_t lds, int32_t has_s,
                                      const float *k, const float *pdef, const float *alpha, const int32_t *prev,
                                      const int32_t *usrc, const float *u, int64_t ldu, const float *hprev,
                                      int64_t ldp, float h_max, float *h, int64_t ldh, void *stream) {
  return guard([&] {
    FLY_REQUIRE(rows >= 0 && batch >= 0 && rows < (int64_t)1 << 30, "size out of range");
    if (!rows || !batch) return;
    FLY_REQUIRE(s_y && lds >= batch && k && pdef && alpha && h && ldh >= batch, "bad argument");
    FLY_REQUIRE(!usrc || (u && ldu >= batch), "input rows need u");
    FLY_REQUIRE(!prev || (hprev && ldp >= batch), "carried rows need the previous state");
    LaunchTimer timer(FLY_K_OTHER, as_stream(stream));
    StepFwdArgs a{s_y, lds, k, pdef, alpha, prev, usrc, u, ldu, hprev, ldp, h, ldh, h_max, (int32_t)rows,
                  (int32_t)batch, has_s != 0};
    const bool v4 = batch % 4 == 0 && vec4_ok(s_y, lds) && vec4_ok(h, ldh) && (!usrc || vec4_ok(u, ldu)) &&
                    (!prev || vec4_ok(hprev, ldp));
    const dim3 grid(blocks_for(rows, 4)), block(256);
    if (v4)
      hipLaunchKernelGGL(k_train_fwd<4>, grid, block, 0, as_stream(stream), a);
    else
      hipLaunchKernelGGL(k_train_fwd<1>, grid, block, 0, as_stream(stream), a);
    check_launch("train step forward");
  });
}

extern "C" int fly_train_step_backward(int64_t rows, int64_t batch, const float *g, int64_t ldg, const float *y,
                                       int64_t ldy, const float *pdef, const float *alpha, const int32_t *prev,
                                       const int32_t *usrc, const float *hprev, int64_t ldp, float h_max, float *gy,
                                       int64_t ldgy, float *gk, float *ga, float *gpdef, float *gu, int64_t ldgu,
                                       float *ghprev, int64_t ldgh, void *stream) {
  return guard([&] {
    FLY_REQUIRE(rows >= 0 && batch >= 0 && rows < (int64_t)1 << 30, "size out of range");
    if (!rows) return;
    FLY_REQUIRE(g && y && pdef && alpha && gy && gk && ga && gpdef, "bad argument");
    FLY_REQUIRE(ldg >= batch && ldy >= batch && ldgy >= batch, "bad leading dimension");
    FLY_REQUIRE(!usrc || (gu && ldgu >= batch), "input rows need gu");
    FLY_REQUIRE(!prev || (hprev && ghprev && ldp >= batch && ldgh >= batch), "carried rows need the previous state");
    LaunchTimer timer(FLY_K_OTHER, as_stream(stream));
    StepBwdArgs a{g, ldg, y, ldy, pdef, alpha, prev, usrc, hprev, ldp, gy, ldgy, gk, ga, gpdef, gu, ldgu, ghprev,
                  ldgh, h_max, (int32_t)rows, (int32_t)batch};
    const bool v4 = batch % 4 == 0 && vec4_ok(g, ldg) && vec4_ok(y, ldy) && vec4_ok(gy, ldgy) &&
                    (!usrc || vec4_ok(gu, ldgu)) && (!prev || (vec4_ok(hprev, ldp) && vec4_ok(ghprev, ldgh)));
    const dim3 grid(blocks_for(rows, 4)), block(256);
    if (v4)
      hipLaunchKernelGGL(k_train_bwd<4>, grid, block, 0, as_stream(stream), a);
    else
      hipLaunchKernelGGL(k_train_bwd<1>, grid, block, 0, as_stream(stream), a);
    check_launch("train step backward");
  });
}

extern "C" int fly_transposed_backward(const int32_t *t_rowptr, const int32_t *t_col, const float *vals,
                                       const int32_t *ids, int64_t nnz, int64_t nrows, int64_t ncols,
                                       const float *gy, int64_t ldgy, const float *h, int64_t ldh, int64_t batch,
                                       float *gh, int64_t ldgh, int32_t accumulate, float *gw, int64_t n_w,
                                       const int32_t *items, int64_t n_items, const int32_t *splits,
                                       int64_t n_splits, float *partials, int64_t n_slots, float *dots,
                                       int64_t n_dots, void *stream) {
  return guard([&] {
    FLY_REQUIRE(nrows >= 0 && ncols >= 0 && batch >= 0, "negative size");
    FLY_REQUIRE(nrows < (int64_t)1 << 24 && ncols < (int64_t)1 << 24, "more than 2^24 rows or columns");
    if (!nrows || !batch) return;
    FLY_REQUIRE(t_rowptr && t_col && vals && ids && gw && h && gh, "bad argument");
    FLY_REQUIRE(batch % 4 == 0 && vec4_ok(h, ldh) && vec4_ok(gh, ldgh) && vec4_ok(gy, ldgy) && ldh >= batch &&
                    ldgh >= batch && ldgy >= batch && ldgy < (1 << 22),
                "the fused backward needs a batch that is a multiple of 4 and 16-byte aligned rows");
    FLY_REQUIRE(ncols == 0 || gy, "bad argument");
    FLY_REQUIRE(nnz >= 0 && nnz < (int64_t)1 << 30 && n_w >= 0 && n_w < (int64_t)1 << 32, "nnz or n_w out of range");
    LaunchTimer timer(FLY_K_OTHER, as_stream(stream));
    FLY_REQUIRE(!items || (n_items >= 0 && n_items < (int64_t)1 << 30 && n_slots >= 0 && n_slots < (int64_t)1 << 30 &&
                           n_splits >= 0 && n_splits <= n_slots && aligned(items, 16)),
                "bad work list");
    FLY_REQUIRE(!items || n_slots == 0 || (partials && splits && vec4_ok(partials, ldgh) && aligned(splits, 16)),
                "a work list with split rows needs partials and splits");
    TransposedArgs a{t_rowptr, t_col, vals, ids, gy, h, gh, gw, ldgy, ldh, ldgh,
                     ncols ? checked_bytes(ncols, ldgy) : 0u, (int32_t)nrows, (int32_t)batch, accumulate != 0,
                     (int32_t)nnz, (uint32_t)n_w, reinterpret_cast<const int4 *>(items),
                     items ? (int32_t)n_items : 0, items ? (int32_t)n_slots : 0, partials};
    const int64_t units = items ? n_items : nrows, chunks = (batch + 63) / 64;
    if (dots) {
      FLY_REQUIRE(n_dots >= chunks * nnz, "dots must hold ceil(batch / 64) * nnz floats");
      FLY_REQUIRE(units * chunks < (int64_t)1 << 31, "chunk-major grid too large");
    }
    if (dots && units) {
      hipLaunchKernelGGL(k_transposed_backward_chunks, dim3(blocks_for(units * chunks, 4)), dim3(256), 0,
                         as_stream(stream), a, dots);
      check_launch("transposed backward (chunks)");
      if (nnz) {
        hipLaunchKernelGGL(k_dots_to_gw, dim3(blocks_for(nnz, 256)), dim3(256), 0, as_stream(stream), dots,
                           (int32_t)nnz, (int32_t)chunks, ids, (uint32_t)n_w, gw);
        check_launch("dots to gw");
      }
    } else if (units) {
      hipLaunchKernelGGL(k_transposed_backward, dim3(blocks_for(units, 4)), dim3(256), 0, as_stream(stream), a);
      check_launch("transposed backward");
    }
    if (items && n_splits > 0) {
      hipLaunchKernelGGL(k_add_partials, dim3(blocks_for(n_splits, 4)), dim3(256), 0, as_stream(stream),
                         reinterpret_cast<const int4 *>(splits), (int32_t)n_splits, partials, (int32_t)n_slots, gh,
                         ldgh, (int32_t)nrows, (int32_t)batch);
      check_launch("partials");
    }
  });
}
