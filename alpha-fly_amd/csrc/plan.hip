// Weight-set plan: everything forward_io needs that depends only on the weights, built once per
// weight version on the device.
//   resting trajectory  c_0 = 0, k_full_t = (t > 1 ? W c_{t-1} : 0) + b, c_t = lerp(c_{t-1}, clamp(k_full_t, 0, H), alpha)
//   deviation mode      lo = -k, hi = H - k, e = k - clamp(k, 0, H), a = alpha, k = k_full_t[R_t]   (brain.py:257-270)
//   float32 mode        k_t = k_full_t[R_t] - A_t c_{t-1}[R_{t-1}], p_default = c_{t-1}[R_t]      (brain.py:238-252, 303-304)
//   sub-matrices        {local column, float32 weight} pairs in W's edge order
#include "common.hpp"
#include "step_kernels.hpp"

#include <algorithm>
#include <memory>

namespace fly {
void validate_graph(int64_t n, int64_t n_edges, const int32_t *crow, const int32_t *pre, hipStream_t st);

namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ float clampf(float x, float lo, float hi) { return fminf(fmaxf(x, lo), hi); }

__global__ void k_edge_weights(const float *__restrict__ sign, const float *__restrict__ w0,
                               const float *__restrict__ lg, int64_t n_edges, float *__restrict__ w) {
  const int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (e < n_edges) w[e] = (sign[e] * w0[e]) * expf(lg[e]);
}

__global__ void k_sigmoid(const float *__restrict__ x, int64_t n, float *__restrict__ y) {
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i < n) y[i] = 1.0f / (1.0f + expf(-x[i]));
}

// Sum over row r's edges of w_e c[pre_e]: 16 lanes per row (a unit), four units per wave.  Lane s of the unit takes
// the edges s, s + 16, ... in rounds of 64 (four loads in flight), and the 16 partial sums meet through xor
// shuffles: the summation order of the training side's one-column products (k_spmv), so the resting trajectory
// has the same bits in both.  A hub row of thousands of partners takes a few hundred rounds instead of thousands
// of dependent loads in one lane.  Every lane of the unit returns the sum.
__device__ __forceinline__ float unit_row_dot(const int32_t *__restrict__ pre, const float *__restrict__ w,
                                              const float *__restrict__ c, int32_t beg, int32_t end, int s) {
  float acc = 0.0f;
  for (int32_t e0 = beg + s; e0 < end; e0 += 64) {
    float v[4], xv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int32_t e = e0 + 16 * j;
      const bool live = e < end;
      v[j] = live ? w[e] : 0.0f;
      xv[j] = live ? c[pre[e]] : 0.0f;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) acc = fmaf(v[j], xv[j], acc);
  }
  acc += __shfl_xor(acc, 8);
  acc += __shfl_xor(acc, 4);
  acc += __shfl_xor(acc, 2);
  acc += __shfl_xor(acc, 1);
  return acc;
}

// k_full[r] = (c ? sum_e w_e c[pre_e] : 0) + bias[r]: one 16-lane unit per row (unit_row_dot)
__global__ __launch_bounds__(256) void k_drive(const int32_t *__restrict__ crow, const int32_t *__restrict__ pre,
                                               const float *__restrict__ w, const float *__restrict__ c,
                                               const float *__restrict__ bias, int64_t n, float *__restrict__ k_full) {
  const int s = threadIdx.x & 15;
  const int64_t r = blockIdx.x * 16 + (threadIdx.x >> 4);
  const bool has = r < n;
  const float sum = has && c ? unit_row_dot(pre, w, c, crow[r], crow[r + 1], s) : 0.0f;
  if (has && s == 0) k_full[r] = sum + bias[r];
}

__global__ void k_rest_update(const float *__restrict__ c, const float *__restrict__ k_full,
                              const float *__restrict__ alpha, float h_max, int64_t n, float *__restrict__ c_next) {
  const int64_t r = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (r < n) c_next[r] = lerp_torch(c ? c[r] : 0.0f, clampf(k_full[r], 0.0f, h_max), alpha[r]);
}

__global__ void k_params_deviation(const int32_t *__restrict__ rows, int64_t nr, const float *__restrict__ k_full,
                                   const float *__restrict__ alpha, float h_max, const int32_t *__restrict__ prev,
                                   const int32_t *__restrict__ usrc, RowParam *__restrict__ rp) {
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i >= nr) return;
  const int32_t r = rows[i];
  const float k = k_full[r];
  RowParam p;
  p.k = 0.0f;
  p.lo = -k;
  p.hi = h_max - k;
  p.e = k - clampf(k, 0.0f, h_max);
  p.a = alpha[r];
  p.pdef = 0.0f;
  p.prev = prev[i];
  p.usrc = usrc[i];
  rp[i] = p;
}

// k_t = k_full[R_t[i]] - sum over the kept edges of w_e c_{t-1}[pre_e]: one 16-lane unit per row of R_t, lane s
// taking the kept edges s, s + 16, ... (as unit_row_dot, through the edge ids)
__global__ __launch_bounds__(256) void k_params_f32(const int32_t *__restrict__ rows, int64_t nr,
                                                    const float *__restrict__ k_full, const float *__restrict__ alpha,
                                                    float h_max, const float *__restrict__ c_prev,
                                                    const int32_t *__restrict__ rowptr,
                                                    const int32_t *__restrict__ edge, const int32_t *__restrict__ pre,
                                                    const float *__restrict__ w, const int32_t *__restrict__ prev,
                                                    const int32_t *__restrict__ usrc, RowParam *__restrict__ rp) {
  const int s = threadIdx.x & 15;
  const int64_t i = blockIdx.x * 16 + (threadIdx.x >> 4);
  const bool has = i < nr;
  float sub = 0.0f;
  if (has && rowptr) {
    const int32_t end = rowptr[i + 1];
    for (int32_t q0 = rowptr[i] + s; q0 < end; q0 += 64) {
      float v[4], xv[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int32_t q = q0 + 16 * j;
        const int32_t e = q < end ? edge[q] : -1;
        v[j] = e >= 0 ? w[e] : 0.0f;
        xv[j] = e >= 0 ? c_prev[pre[e]] : 0.0f;
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) sub = fmaf(v[j], xv[j], sub);
    }
  }
  sub += __shfl_xor(sub, 8);
  sub += __shfl_xor(sub, 4);
  sub += __shfl_xor(sub, 2);
  sub += __shfl_xor(sub, 1);
  if (!has || s != 0) return;
  const int32_t r = rows[i];
  RowParam p;
  p.k = k_full[r] - sub;
  p.lo = 0.0f;
  p.hi = h_max;
  p.e = 0.0f;
  p.a = alpha[r];
  p.pdef = c_prev ? c_prev[r] : 0.0f;
  p.prev = prev[i];
  p.usrc = usrc[i];
  rp[i] = p;
}

__global__ void k_params_full(const float *__restrict__ alpha, float h_max, int64_t n, RowParam *__restrict__ rp) {
  const int64_t r = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (r >= n) return;
  RowParam p;
  p.k = 0.0f;
  p.lo = 0.0f;
  p.hi = h_max;
  p.e = 0.0f;
  p.a = alpha[r];
  p.pdef = 0.0f;
  p.prev = (int32_t)r;
  p.usrc = (int32_t)r;
  rp[r] = p;
}

__global__ void k_pack(const int32_t *__restrict__ col, const int32_t *__restrict__ edge, const float *__restrict__ w,
                       int64_t nnz, int2 *__restrict__ cv) {
  const int64_t q = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (q >= nnz) return;
  const int32_t e = edge ? edge[q] : (int32_t)q;
  cv[q] = make_int2(col[q], __float_as_int(w[e]));
}

__global__ void k_unpack(const int2 *__restrict__ cv, int64_t nnz, int32_t *__restrict__ col, float *__restrict__ val) {
  const int64_t q = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (q >= nnz) return;
  const int2 p = cv[q];
  if (col) col[q] = p.x;
  if (val) val[q] = __int_as_float(p.y);
}

// c_out[j] = c_T[out_idx[j]]; cbase is what the head adds to the carried state at output j: the resting
// value in deviation mode, and in float32 mode the resting value only where the output is not carried.
__global__ void k_out_base(const int32_t *__restrict__ out_idx, const int32_t *__restrict__ out_src,
                           const float *__restrict__ c_last, int64_t n_out, int32_t mode, float *__restrict__ c_out,
                           float *__restrict__ cbase) {
  const int64_t j = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (j >= n_out) return;
  const float c = c_last ? c_last[out_idx[j]] : 0.0f;
  c_out[j] = c;
  cbase[j] = (mode == FLY_MODE_F32 && out_src[j] >= 0) ? 0.0f : c;
}

}  // namespace

// The tables of step t of the cone under cfg: built on the first plan that asks and kept on the cone, since they
// depend on the structure only (null when the step does not sweep).  Guarded by the cache's lock.
std::shared_ptr<const SweepTables> cone_sweep(const fly_cone &cone, int t, const SweepConfig &cfg, hipStream_t st) {
  ConeSweepCache &c = *cone.sweep_cache;
  std::lock_guard<std::mutex> lock(c.mu);
  for (const auto &e : c.entries)
    if (e.t == t && e.cfg == cfg) return e.tables;
  std::shared_ptr<const SweepTables> tables =
      build_sweep<int32_t>(cone.rowptr[t].p, cone.col[t].p, cone.rows_n[t], cone.nnz[t], cone.rows_n[t - 1], cfg, st);
  c.entries.push_back({t, cfg, tables});
  return tables;
}

}  // namespace fly

using namespace fly;

extern "C" int fly_edge_weights(const float *sign, const float *w0, const float *log_gain, int64_t n_edges, float *w,
                                void *stream) {
  return guard([&] {
    FLY_REQUIRE(n_edges >= 0, "negative n_edges");
    if (!n_edges) return;
    FLY_REQUIRE(sign && w0 && log_gain && w, "null argument");
    hipLaunchKernelGGL(k_edge_weights, dim3(blocks_for(n_edges, kThreads)), dim3(kThreads), 0, as_stream(stream), sign,
                       w0, log_gain, n_edges, w);
    check_launch("edge weights");
  });
}

extern "C" int fly_plan_create(const fly_cone *cone, const int32_t *crow, const int32_t *pre, const float *w,
                               const float *bias, const float *alpha_logit, float h_max, int32_t mode, void *stream,
                               fly_plan **out) {
  return guard([&] {
    FLY_REQUIRE(out != nullptr, "out is null");
    *out = nullptr;
    FLY_REQUIRE(cone != nullptr, "cone is null");
    FLY_REQUIRE(mode == FLY_MODE_DEVIATION_F16 || mode == FLY_MODE_F32, "unknown mode");
    FLY_REQUIRE(h_max >= 0.0f, "h_max must be >= 0 (+inf: no upper clamp)");
    FLY_REQUIRE(crow && bias && alpha_logit && (cone->n_edges == 0 || (pre && w)), "null argument");
    FLY_REQUIRE(current_device() == cone->device, "the cone lives on another device");
    hipStream_t st = as_stream(stream);
    const int64_t n = cone->n;
    const int T = cone->steps;
    const unsigned nb = blocks_for(n, kThreads);
    validate_graph(n, cone->n_edges, crow, pre, st);

    auto plan = std::make_unique<fly_plan>();
    plan->device = cone->device;
    plan->mode = mode;
    plan->steps = T;
    plan->h_max = h_max;
    plan->n = n;
    plan->n_in = cone->n_in;
    plan->n_out = cone->n_out;
    plan->rows_n = cone->rows_n;
    plan->nnz = cone->nnz;
    plan->max_rows = 0;
    for (int t = 1; t <= T; ++t) plan->max_rows = std::max(plan->max_rows, cone->rows_n[t]);
    plan->rowptr.resize(T + 1);
    plan->colval.resize(T + 1);
    plan->params.resize(T + 1);
    plan->sweep.resize(T + 1);
    plan->lead.resize(T + 1);
    plan->lead_flag.resize(T + 1);
    plan->nlead.assign(T + 1, 0);
    plan->tune = tuning_snapshot();
    const SweepConfig cfg = sweep_config(plan->tune);

    DevArray<float> alpha(n), k_full(n), c_a(n), c_b(n);
    hipLaunchKernelGGL(k_sigmoid, dim3(nb), dim3(kThreads), 0, st, alpha_logit, n, alpha.p);
    float *c_prev = nullptr;  // c_0 = 0
    float *c_next = c_a.p;
    for (int t = 1; t <= T; ++t) {
      hipLaunchKernelGGL(k_drive, dim3(blocks_for(n, 16)), dim3(256), 0, st, crow, pre, w, t > 1 ? c_prev : nullptr,
                         bias, n, k_full.p);
      const int64_t nr = cone->rows_n[t];
      plan->params[t].alloc(nr);
      if (cone->has_op[t]) {
        plan->rowptr[t].alloc(nr + 1);
        FLY_HIP(hipMemcpyAsync(plan->rowptr[t].p, cone->rowptr[t].p, sizeof(int32_t) * (nr + 1), hipMemcpyDeviceToDevice, st));
        plan->colval[t].alloc(cone->nnz[t]);
        if (cone->nnz[t])
          hipLaunchKernelGGL(k_pack, dim3(blocks_for(cone->nnz[t], kThreads)), dim3(kThreads), 0, st, cone->col[t].p,
                             cone->edge[t].p, w, cone->nnz[t], plan->colval[t].p);
        if (plan->tune.swept >= 0) {
          plan->sweep[t] = cone_sweep(*cone, t, cfg, st);
          if (plan->sweep[t]) plan->max_pieces = std::max(plan->max_pieces, plan->sweep[t]->pieces);
        }
        if (cone->nnz[t] < 16 * nr) {   // short rows on average: the step runs as row slots
          LeadSlots ls = build_lead_slots(plan->rowptr[t].p, nr, cone->nnz[t], st);
          plan->lead[t] = std::move(ls.lead);
          plan->lead_flag[t] = std::move(ls.flag);
          plan->nlead[t] = ls.n;
        }
      }
      if (nr) {
        if (mode == FLY_MODE_DEVIATION_F16)
          hipLaunchKernelGGL(k_params_deviation, dim3(blocks_for(nr, kThreads)), dim3(kThreads), 0, st, cone->rows[t].p,
                             nr, k_full.p, alpha.p, h_max, cone->prev[t].p, cone->usrc[t].p, plan->params[t].p);
        else
          hipLaunchKernelGGL(k_params_f32, dim3(blocks_for(nr, 16)), dim3(256), 0, st, cone->rows[t].p, nr,
                             k_full.p, alpha.p, h_max, c_prev, cone->has_op[t] && c_prev ? cone->rowptr[t].p : nullptr,
                             cone->edge[t].p, pre, w, cone->prev[t].p, cone->usrc[t].p, plan->params[t].p);
      }
      hipLaunchKernelGGL(k_rest_update, dim3(nb), dim3(kThreads), 0, st, c_prev, k_full.p, alpha.p, h_max, n, c_next);
      c_prev = c_next;
      c_next = (c_next == c_a.p) ? c_b.p : c_a.p;
    }
    plan->out_src.alloc(cone->n_out);
    plan->cbase.alloc(cone->n_out);
    plan->c_out.alloc(cone->n_out);
    if (cone->n_out) {
      FLY_HIP(hipMemcpyAsync(plan->out_src.p, cone->out_src.p, sizeof(int32_t) * cone->n_out, hipMemcpyDeviceToDevice, st));
      hipLaunchKernelGGL(k_out_base, dim3(blocks_for(cone->n_out, kThreads)), dim3(kThreads), 0, st, cone->out_idx.p,
                         cone->out_src.p, c_prev, cone->n_out, mode, plan->c_out.p, plan->cbase.p);
    }
    check_launch("plan");
    FLY_HIP(hipStreamSynchronize(st));
    *out = plan.release();
  });
}

extern "C" int fly_plan_create_full(int64_t n, int64_t n_edges, const int32_t *crow, const int32_t *pre, const float *w,
                                    const float *alpha_logit, float h_max, const fly_sweep *sweep, void *stream,
                                    fly_plan **out) {
  return guard([&] {
    FLY_REQUIRE(out != nullptr, "out is null");
    *out = nullptr;
    FLY_REQUIRE(n > 0 && n < (int64_t)INT32_MAX && n_edges >= 0 && n_edges < (int64_t)INT32_MAX, "size out of range");
    FLY_REQUIRE(crow && alpha_logit && (n_edges == 0 || (pre && w)), "null argument");
    FLY_REQUIRE(h_max >= 0.0f, "h_max must be >= 0 (+inf: no upper clamp)");
    hipStream_t st = as_stream(stream);
    validate_graph(n, n_edges, crow, pre, st);
    auto plan = std::make_unique<fly_plan>();
    plan->device = current_device();
    plan->mode = FLY_MODE_F32;
    plan->full = true;
    plan->steps = 0;
    plan->h_max = h_max;
    plan->n = n;
    plan->n_in = n;
    plan->n_out = n;
    plan->max_rows = n;
    plan->rows_n = {n};
    plan->nnz = {n_edges};
    plan->rowptr.resize(1);
    plan->colval.resize(1);
    plan->params.resize(1);
    plan->rowptr[0].alloc(n + 1);
    FLY_HIP(hipMemcpyAsync(plan->rowptr[0].p, crow, sizeof(int32_t) * (n + 1), hipMemcpyDeviceToDevice, st));
    plan->colval[0].alloc(n_edges);
    if (n_edges)
      hipLaunchKernelGGL(k_pack, dim3(blocks_for(n_edges, kThreads)), dim3(kThreads), 0, st, pre, nullptr, w, n_edges,
                         plan->colval[0].p);
    DevArray<float> alpha(n);
    hipLaunchKernelGGL(k_sigmoid, dim3(blocks_for(n, kThreads)), dim3(kThreads), 0, st, alpha_logit, n, alpha.p);
    plan->params[0].alloc(n);
    hipLaunchKernelGGL(k_params_full, dim3(blocks_for(n, kThreads)), dim3(kThreads), 0, st, alpha.p, h_max, n,
                       plan->params[0].p);
    plan->tune = tuning_snapshot();
    plan->sweep.resize(1);
    plan->lead.resize(1);
    plan->lead_flag.resize(1);
    plan->nlead.assign(1, 0);
    if (sweep && sweep->t && plan->tune.swept >= 0) {
      FLY_REQUIRE(sweep->device == plan->device, "the sweep tables live on another device");
      FLY_REQUIRE(sweep->t->nrows == n && sweep->t->ncols == n && sweep->t->nnz == n_edges,
                  "the sweep tables belong to another structure");
      plan->sweep[0] = sweep->t;
      plan->max_pieces = sweep->t->pieces;
    }
    check_launch("full plan");
    FLY_HIP(hipStreamSynchronize(st));
    *out = plan.release();
  });
}

extern "C" int fly_plan_destroy(fly_plan *plan) {
  return guard([&] { delete plan; });
}

extern "C" int fly_plan_resting(const fly_plan *plan, float *c_out, void *stream) {
  return guard([&] {
    FLY_REQUIRE(plan && c_out, "null argument");
    FLY_REQUIRE(!plan->full, "the literal-recurrence plan has no resting outputs");
    if (plan->n_out)
      FLY_HIP(hipMemcpyAsync(c_out, plan->c_out.p, sizeof(float) * plan->n_out, hipMemcpyDeviceToDevice, as_stream(stream)));
  });
}

extern "C" int fly_plan_matrix(const fly_plan *plan, int32_t t, int32_t *rowptr, int32_t *col, float *val,
                               void *stream) {
  return guard([&] {
    FLY_REQUIRE(plan != nullptr, "plan is null");
    FLY_REQUIRE(current_device() == plan->device, "the plan lives on another device");
    FLY_REQUIRE(plan->full ? t == 1 : (t >= 1 && t <= plan->steps), "step out of range");
    const int ti = plan->full ? 0 : t;
    if (plan->rowptr[ti].p == nullptr) return;   // A_t does not exist (R_{t-1} is empty)
    hipStream_t st = as_stream(stream);
    const int64_t nr = plan->rows_n[ti], nnz = plan->nnz[ti];
    if (rowptr)
      FLY_HIP(hipMemcpyAsync(rowptr, plan->rowptr[ti].p, sizeof(int32_t) * (nr + 1), hipMemcpyDeviceToDevice, st));
    if (nnz && (col || val)) {
      hipLaunchKernelGGL(k_unpack, dim3(blocks_for(nnz, kThreads)), dim3(kThreads), 0, st, plan->colval[ti].p, nnz,
                         col, val);
      check_launch("plan matrix");
    }
  });
}

extern "C" int fly_sweep_create(const int32_t *rowptr, const int32_t *col, int64_t nrows, int64_t nnz, int64_t ncols,
                                void *stream, fly_sweep **out) {
  return guard([&] {
    FLY_REQUIRE(out != nullptr, "out is null");
    *out = nullptr;
    FLY_REQUIRE(nrows >= 0 && nnz >= 0 && ncols >= 0, "negative size");
    FLY_REQUIRE(rowptr && (nnz == 0 || col), "null argument");
    auto sw = std::make_unique<fly_sweep>();
    sw->device = current_device();
    sw->tune = tuning_snapshot();
    if (sw->tune.swept < 0) return;   // the sweep is off: nothing to build
    sw->t = build_sweep<int32_t>(rowptr, col, nrows, nnz, ncols, sweep_config(sw->tune), as_stream(stream));
    if (sw->t) *out = sw.release();
  });
}

extern "C" int fly_sweep_destroy(fly_sweep *sweep) {
  return guard([&] { delete sweep; });
}

extern "C" int fly_sweep_info(const fly_sweep *sweep, int64_t *info) {
  return guard([&] {
    FLY_REQUIRE(sweep && sweep->t && info, "null argument");
    const SweepTables &t = *sweep->t;
    info[0] = t.npos;
    info[1] = t.pieces;
    info[2] = t.split_rows;
    info[3] = t.rows_per_wave;
    info[4] = t.bands;
    info[5] = t.grid;
    info[6] = (int64_t)reinterpret_cast<uintptr_t>(t.order.p);
  });
}

extern "C" int fly_plan_sweep_info(const fly_plan *plan, int32_t t, int64_t *info) {
  return guard([&] {
    FLY_REQUIRE(plan && info, "null argument");
    FLY_REQUIRE(plan->full ? t == 1 : (t >= 1 && t <= plan->steps), "step out of range");
    const SweepTables *s = plan->sweep[plan->full ? 0 : t].get();
    for (int i = 0; i < 7; ++i) info[i] = 0;
    if (!s) return;
    info[0] = s->npos;
    info[1] = s->pieces;
    info[2] = s->split_rows;
    info[3] = s->rows_per_wave;
    info[4] = s->bands;
    info[5] = s->grid;
    info[6] = (int64_t)reinterpret_cast<uintptr_t>(s->order.p);
  });
}
