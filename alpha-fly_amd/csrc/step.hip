// The recurrent state step's launches, and the forward_io / literal / per-step drivers of the evaluator.
//
// One pass per step fuses the reference's SpMM, index_add_, gather and jiterator update
// (chessfly/brain.py:273-277, 310-313, 217-223); the kernels and their launch shapes are in step_kernels.hpp.
#include <cmath>
#include <cstring>
#include <mutex>
#include <type_traits>

#include "step_kernels.hpp"

namespace fly {

namespace {
std::mutex g_tuning_mu;
Tuning g_tuning;   // the defaults fly_set_tuning sets
}  // namespace

Tuning tuning_snapshot() {
  std::lock_guard<std::mutex> lock(g_tuning_mu);
  return g_tuning;
}

namespace {

// Deviation mode (half state) updates with p + a (x - p) like the reference's fused kernel; float32 mode
// with torch.lerp's formula, like the reference's CPU path.
template <typename S, typename U, int V>
void launch_v(const StepArgs<S, U> &a, int groups, int unroll, bool rows_mode, int step_lds, hipStream_t st) {
  const int64_t waves = (int64_t)a.slots * a.wpt * a.ntiles + (int64_t)a.nlead * a.ntiles;   // lead slots first
  FLY_REQUIRE(waves < (int64_t)UINT32_MAX / 2, "state step grid too large");
  const dim3 grid(blocks_for(waves, 4)), block(256);
  LaunchTimer timer(FLY_K_STATE_STEP, st);
  constexpr bool kTL = sizeof(S) == 4;
  // the kernels use no LDS: a reservation only caps the workgroups (waves per SIMD) a CU runs at once
  const unsigned lds = (unsigned)std::max(0, step_lds);
  if constexpr (V * sizeof(S) == 32) {
    // 32-byte lanes exist for the row slots of half states only (state_step picks them for nothing else)
    hipLaunchKernelGGL((k_state_step_rows<S, U, V, 8, 4, kTL>), grid, block, lds, st, a);
    return;
  }
  if constexpr (V * sizeof(S) == 16) {
    if (rows_mode) {
      if (unroll <= 4) {   // 4 measured best for the row slots
        if (groups == 8) hipLaunchKernelGGL((k_state_step_rows<S, U, V, 8, 4, kTL>), grid, block, lds, st, a);
        else if (groups == 4) hipLaunchKernelGGL((k_state_step_rows<S, U, V, 4, 4, kTL>), grid, block, lds, st, a);
        else hipLaunchKernelGGL((k_state_step_rows<S, U, V, 2, 4, kTL>), grid, block, lds, st, a);
      } else {
        if (groups == 8) hipLaunchKernelGGL((k_state_step_rows<S, U, V, 8, 8, kTL>), grid, block, lds, st, a);
        else if (groups == 4) hipLaunchKernelGGL((k_state_step_rows<S, U, V, 4, 8, kTL>), grid, block, lds, st, a);
        else hipLaunchKernelGGL((k_state_step_rows<S, U, V, 2, 8, kTL>), grid, block, lds, st, a);
      }
      return;
    }
    if (groups == 8) {
      hipLaunchKernelGGL((k_state_step_grouped<S, U, V, 8, 4, kTL>), grid, block, lds, st, a);
      return;
    }
    if (groups == 4) {
      hipLaunchKernelGGL((k_state_step_grouped<S, U, V, 4, 8, kTL>), grid, block, lds, st, a);
      return;
    }
    if (groups == 2) {
      hipLaunchKernelGGL((k_state_step_grouped<S, U, V, 2, 8, kTL>), grid, block, lds, st, a);
      return;
    }
  }
  if (unroll >= 32)
    hipLaunchKernelGGL((k_state_step<S, U, V, 32, kTL>), grid, block, lds, st, a);
  else if (unroll >= 16)   // 8 (also for 0) measured best for one non-zero per wave
    hipLaunchKernelGGL((k_state_step<S, U, V, 16, kTL>), grid, block, lds, st, a);
  else
    hipLaunchKernelGGL((k_state_step<S, U, V, 8, kTL>), grid, block, lds, st, a);
}

// One state step.  `sweep`: the step matrix's banded-sweep tables (null: the step does not sweep); a.pieces must then
// hold sweep_pieces_bytes(sweep, batch) bytes.
template <typename S, typename U>
void state_step(StepArgs<S, U> a, double avg_nnz, const Tuning &tune, const SweepTables *sweep, hipStream_t st) {
  if (a.nrows == 0 || a.batch == 0) return;
  Tuning tu = tune;
  if (sweep && tune.swept > 0) tu.rows_mode = -1;   // a forced sweep takes steps of short rows too
  const StepShape sh = shape_step(a, avg_nnz, tu);
  const int v = sh.v, groups = sh.groups, unroll = sh.unroll;
  const bool rows_mode = sh.rows_mode;
  // lead slots are tables of slots of 8 rows, taken one chunk per tile
  if (!(rows_mode && groups == 8 && a.wpt == 1 && a.lead && a.lead_flag && a.slots == (a.nrows + 7) / 8)) {
    a.lead = nullptr;
    a.lead_flag = nullptr;
    a.nlead = 0;
  }
  // long-row steps with sweep tables: the banded sweep, on the grouped kernel's lane layout
  if (sweep && tune.swept >= 0 && v == 16 / (int)sizeof(S) && groups == 8 && !rows_mode && a.rowptr && a.xprev &&
      a.xbytes && !(a.out_exact && a.batch % v)) {
    LaunchTimer timer(FLY_K_STATE_STEP, st);
    a.sweep_paired = tune.sweep_paired;
    a.sweep_slots = tune.sweep_slots;
    a.sweep_pipe = tune.sweep_pipe;
    a.sweep_last_sync = tune.sweep_last_sync;
    launch_swept<S, U, 0>(a, *sweep, st);
    check_launch("swept state step");
    return;
  }
  switch (v) {
    // only 16-byte lanes (V = 16 / sizeof(S)) have grouped and row-slot kernels, and 32-byte lanes of half
    // states a row-slot kernel; pick_shape sets groups to 1 for every other V, so rows_mode is false there too
    case 1: launch_v<S, U, 1>(a, 1, unroll, false, tune.step_lds, st); break;
    case 2: launch_v<S, U, 2>(a, 1, unroll, false, tune.step_lds, st); break;
    case 4: launch_v<S, U, 4>(a, groups, unroll, rows_mode, tune.step_lds, st); break;
    case 8:
      if constexpr (sizeof(S) == 2) launch_v<S, U, 8>(a, groups, unroll, rows_mode, tune.step_lds, st);
      break;
    default:
      if constexpr (sizeof(S) == 2) launch_v<S, U, 16>(a, groups, unroll, rows_mode, tune.step_lds, st);
      break;
  }
  check_launch("state step");
}

// Row-looped 2-D launches: blockIdx.x covers the batch, blockIdx.y strides over the rows.
inline dim3 rows_grid(int64_t rows, int64_t batch) {
  return dim3(blocks_for(batch, 256), (unsigned)std::max<int64_t>(1, std::min<int64_t>(rows, 65535)));
}

template <typename S>
__global__ void k_outputs(const S *__restrict__ state, int64_t lds, const int32_t *__restrict__ out_src,
                          const float *__restrict__ cbase, int64_t n_out, int64_t batch, float *__restrict__ out,
                          int64_t ldo) {
  const int64_t b = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (b >= batch) return;
  for (int64_t j = blockIdx.y; j < n_out; j += gridDim.y) {
    const int32_t src = out_src[j];
    const float d = (state != nullptr && src >= 0) ? static_cast<float>(state[(int64_t)src * lds + b]) : 0.0f;
    out[j * ldo + b] = cbase[j] + d;
  }
}

template <typename T>
__global__ void k_add_bias(T *__restrict__ u, int64_t ldu, const float *__restrict__ bias, int64_t n, int64_t batch) {
  const int64_t b = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (b >= batch) return;
  for (int64_t r = blockIdx.y; r < n; r += gridDim.y) u[r * ldu + b] += static_cast<T>(bias[r]);
}

template <typename T>
__global__ void k_zero_rows(T *__restrict__ h, int64_t ld, int64_t n, int64_t batch) {
  const int64_t b = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (b >= batch) return;
  for (int64_t r = blockIdx.y; r < n; r += gridDim.y) h[r * ld + b] = T(0);
}

// One float64 update of the literal recurrence (brain.py:219-220 in u's dtype): per row, the CSR sum in edge
// order, x = clamp(s + drive, 0, H), h' = torch.lerp(h, x, alpha), all in double.  The plan's float32 weights,
// alphas and bound widen exactly, as the reference's .to(u.dtype) does.  One wave per (row, 64 columns), one column
// per lane; the row's pairs are wave-uniform.
__global__ __launch_bounds__(256) void k_literal_step_f64(const int32_t *__restrict__ rowptr, const int2 *__restrict__ colval,
                                                          const RowParam *__restrict__ params, const double *hprev,
                                                          int64_t ldp, const double *__restrict__ drive, int64_t ldd,
                                                          double *__restrict__ hout, int64_t ldo, int32_t nrows,
                                                          int32_t batch, int32_t chunks) {
  const uint32_t wave = blockIdx.x * 4u + (uint32_t)__builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t row = wave / (uint32_t)chunks, chunk = wave - row * (uint32_t)chunks;
  if (row >= (uint32_t)nrows) return;
  const int64_t b = (int64_t)chunk * 64 + (threadIdx.x & 63);
  if (b >= batch) return;
  double acc = 0.0;
  if (hprev != nullptr) {
    const int32_t end = rowptr[row + 1];
    for (int32_t e = rowptr[row]; e < end; ++e) {
      const int2 cv = colval[e];
      acc = fma((double)__int_as_float(cv.y), hprev[(int64_t)cv.x * ldp + b], acc);
    }
  }
  const RowParam p = params[row];
  const double x = fmin(fmax(acc + drive[(int64_t)row * ldd + b], 0.0), (double)p.hi);
  const double h = hprev != nullptr ? hprev[(int64_t)row * ldp + b] : 0.0;
  const double a = (double)p.a;
  hout[(int64_t)row * ldo + b] = fabs(a) < 0.5 ? h + a * (x - h) : x - (x - h) * (1.0 - a);
}

// One float64 step of the light cone (brain.py:307-327 with u_in float64).  The reference builds its cache in
// the parameters' dtype (float32) and widens it with .to(dtype): the float32 plan's k_t, c_{t-1}, alphas and A_t
// values widen exactly here, and the sum, input add, clamp and lerp are double.  The order is the fused update's
// (brain.py:310-313): x = clamp((A_t h + u) + k_t, 0, H), p = carried ? h_{t-1}[prev] : c_{t-1}.  One wave per
// (row, 64 columns), one column per lane; the row's pairs are wave-uniform.
__global__ __launch_bounds__(256) void k_cone_step_f64(const int32_t *__restrict__ rowptr, const int2 *__restrict__ colval,
                                                       const RowParam *__restrict__ params, const double *hprev,
                                                       int64_t ldp, const double *__restrict__ u, int64_t ldu,
                                                       double *__restrict__ hout, int64_t ldo, int32_t nrows,
                                                       int32_t batch, int32_t chunks) {
  const uint32_t wave = blockIdx.x * 4u + (uint32_t)__builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t row = wave / (uint32_t)chunks, chunk = wave - row * (uint32_t)chunks;
  if (row >= (uint32_t)nrows) return;
  const int64_t b = (int64_t)chunk * 64 + (threadIdx.x & 63);
  if (b >= batch) return;
  double acc = 0.0;
  if (hprev != nullptr && rowptr != nullptr) {
    const int32_t end = rowptr[row + 1];
    for (int32_t e = rowptr[row]; e < end; ++e) {
      const int2 cv = colval[e];
      acc = fma((double)__int_as_float(cv.y), hprev[(int64_t)cv.x * ldp + b], acc);
    }
  }
  const RowParam p = params[row];
  if (u != nullptr && p.usrc >= 0) acc += u[(int64_t)p.usrc * ldu + b];
  const double x = fmin(fmax(acc + (double)p.k, (double)p.lo), (double)p.hi) + (double)p.e;
  const double h = (hprev != nullptr && p.prev >= 0) ? hprev[(int64_t)p.prev * ldp + b] : (double)p.pdef;
  const double a = (double)p.a;
  hout[(int64_t)row * ldo + b] = fabs(a) < 0.5 ? h + a * (x - h) : x - (x - h) * (1.0 - a);
}

// out[j] = c_T[out_idx[j]] widened, or the state of out_idx[j] in R_T where it has one (float32 plans carry a
// zero base there).
__global__ void k_outputs_f64(const double *__restrict__ state, int64_t lds, const int32_t *__restrict__ out_src,
                              const float *__restrict__ cbase, int64_t n_out, int64_t batch, double *__restrict__ out,
                              int64_t ldo) {
  const int64_t b = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (b >= batch) return;
  for (int64_t j = blockIdx.y; j < n_out; j += gridDim.y) {
    const int32_t src = out_src[j];
    out[j * ldo + b] = (state != nullptr && src >= 0) ? state[(int64_t)src * lds + b] + (double)cbase[j]
                                                      : (double)cbase[j];
  }
}

}  // namespace

// Boards per block of a forward: the whole batch while a state buffer of `rows` rows stays below 2 GiB, so the
// gathers keep 32-bit buffer offsets; a larger batch runs as equal blocks of whole 64-column chunks that do
// (the boards are independent).
int64_t block_cols(int64_t rows, size_t elem, int64_t batch) {
  auto fits = [&](int64_t b) { return rows == 0 || buffer_bytes(rows, state_ld(b, elem), elem) != 0; };
  for (int64_t n = 1;; ++n) {
    const int64_t b = n == 1 ? batch : round_up((batch + n - 1) / n, 64);
    if (fits(b) || b <= 64) return b;
  }
}

size_t state_bytes(const fly_plan &plan) { return plan.mode == FLY_MODE_DEVIATION_F16 ? 2 : 4; }

int64_t io_block(const fly_plan &plan, int64_t batch) { return block_cols(plan.max_rows, state_bytes(plan), batch); }

size_t plan_pieces_bytes(const fly_plan &plan, int64_t batch) {
  return plan.max_pieces ? align256((size_t)plan.max_pieces * (size_t)round_up(batch, 64) * sizeof(float)) : 0;
}

size_t io_states_bytes(const fly_plan &plan, int64_t blk) {
  const size_t es = state_bytes(plan);
  return align256(2 * (size_t)plan.max_rows * (size_t)state_ld(blk, es) * es + 256);
}

size_t io_workspace(const fly_plan &plan, int64_t batch) {
  const int64_t blk = io_block(plan, batch);
  return io_states_bytes(plan, blk) + plan_pieces_bytes(plan, blk);
}

// Runs steps 1..T of a light-cone plan.  Returns the final state (null if R_T is empty) in one of the two
// workspace buffers, whose row stride is state_ld(batch, sizeof(S)).  u_padded: the drive u is the library's own
// workspace, whose rows may be read up to the batch rounded up to 64 columns.  pieces: plan_pieces_bytes(plan,
// batch) bytes for the sums of split rows.
template <typename S, typename U>
const S *run_cone_steps(const fly_plan &plan, const U *u, int64_t ldu, int64_t batch, bool u_padded, void *ws,
                        float *pieces, hipStream_t st) {
  const int64_t lds = state_ld(batch, sizeof(S));
  S *buf[2] = {reinterpret_cast<S *>(ws), reinterpret_cast<S *>(ws) + (size_t)plan.max_rows * lds};
  const S *prev = nullptr;
  int cur = 0;
  for (int t = 1; t <= plan.steps; ++t) {
    const int64_t nr = plan.rows_n[t];
    if (nr == 0) {
      prev = nullptr;
      continue;
    }
    StepArgs<S, U> a{};
    a.rowptr = plan.rowptr[t].p;  // null where A_t does not exist
    a.colval = plan.colval[t].p;
    a.params = plan.params[t].p;
    a.lead = plan.lead[t].p;
    a.lead_flag = plan.lead_flag[t].p;
    a.nlead = plan.nlead[t];
    a.xprev = prev;
    a.ldx = lds;
    a.u = u;
    a.ldu = ldu;
    a.u_padded = u_padded ? 1 : 0;
    a.xout = buf[cur];
    a.ldo = lds;
    a.nrows = (int32_t)nr;
    a.batch = (int32_t)batch;
    a.xbytes = prev ? buffer_bytes(plan.rows_n[t - 1], lds, sizeof(S)) : 0;
    a.pieces = pieces;
    a.sweep_exact = std::isfinite(plan.h_max) ? 0 : 1;   // no upper clamp: a state may overflow to inf
    state_step(a, nr ? (double)plan.nnz[t] / (double)nr : 0.0, plan.tune, plan.sweep[t].get(), st);
    prev = buf[cur];
    cur ^= 1;
  }
  return prev;
}

template <typename S>
void write_outputs(const fly_plan &plan, const S *state, int64_t batch, float *out, int64_t ldo, hipStream_t st) {
  if (!plan.n_out || !batch) return;
  LaunchTimer timer(FLY_K_OTHER, st);
  hipLaunchKernelGGL(k_outputs<S>, rows_grid(plan.n_out, batch), dim3(256), 0, st, state, state_ld(batch, sizeof(S)),
                     plan.out_src.p, plan.cbase.p,
                     plan.n_out, batch, out, ldo);
  check_launch("outputs");
}

template const _Float16 *run_cone_steps<_Float16, _Float16>(const fly_plan &, const _Float16 *, int64_t, int64_t, bool,
                                                            void *, float *, hipStream_t);
template const _Float16 *run_cone_steps<_Float16, float>(const fly_plan &, const float *, int64_t, int64_t, bool, void *,
                                                         float *, hipStream_t);
template const float *run_cone_steps<float, float>(const fly_plan &, const float *, int64_t, int64_t, bool, void *,
                                                   float *, hipStream_t);

void check_plan_device(const fly_plan *plan) {
  FLY_REQUIRE(plan != nullptr, "plan is null");
  FLY_REQUIRE(current_device() == plan->device, "the plan lives on another device");
}

}  // namespace fly

using namespace fly;

extern "C" size_t fly_forward_io_workspace(const fly_plan *plan, int64_t batch) {
  return plan ? io_workspace(*plan, batch) : 0;
}

extern "C" int fly_forward_io(const fly_plan *plan, const void *u_in, int64_t ldu, int64_t batch, float *out,
                              int64_t ldo, void *ws, size_t ws_bytes, void *stream) {
  return guard([&] {
    check_plan_device(plan);
    FLY_REQUIRE(!plan->full, "forward_io needs a light-cone plan");
    FLY_REQUIRE(batch >= 0 && batch < (int64_t)INT32_MAX / 2, "batch out of range");
    if (batch == 0) return;
    FLY_REQUIRE(out && ldo >= batch, "bad output");
    FLY_REQUIRE(plan->n_in == 0 || (u_in && ldu >= batch), "bad input drive");
    FLY_REQUIRE(ws && ws_bytes >= io_workspace(*plan, batch), "workspace too small");
    FLY_REQUIRE(aligned(ws, 256), "workspace must be 256-byte aligned");
    hipStream_t st = as_stream(stream);
    const int64_t blk = io_block(*plan, batch);
    float *pieces = reinterpret_cast<float *>(static_cast<char *>(ws) + io_states_bytes(*plan, blk));
    for (int64_t c0 = 0; c0 < batch; c0 += blk) {
      const int64_t nb = std::min(blk, batch - c0);
      if (plan->mode == FLY_MODE_DEVIATION_F16) {
        const _Float16 *u = plan->n_in ? static_cast<const _Float16 *>(u_in) + c0 : nullptr;
        const _Float16 *fin = run_cone_steps<_Float16, _Float16>(*plan, u, ldu, nb, false, ws, pieces, st);
        write_outputs<_Float16>(*plan, fin, nb, out + c0, ldo, st);
      } else {
        const float *u = plan->n_in ? static_cast<const float *>(u_in) + c0 : nullptr;
        const float *fin = run_cone_steps<float, float>(*plan, u, ldu, nb, false, ws, pieces, st);
        write_outputs<float>(*plan, fin, nb, out + c0, ldo, st);
      }
    }
  });
}

extern "C" size_t fly_forward_io_f64_workspace(const fly_plan *plan, int64_t batch) {
  if (!plan) return 0;
  return 2 * (size_t)plan->max_rows * (size_t)std::max<int64_t>(batch, 1) * sizeof(double) + 256;
}

extern "C" int fly_forward_io_f64(const fly_plan *plan, const double *u_in, int64_t ldu, int64_t batch, double *out,
                                  int64_t ldo, void *ws, size_t ws_bytes, void *stream) {
  return guard([&] {
    check_plan_device(plan);
    FLY_REQUIRE(!plan->full, "forward_io needs a light-cone plan");
    FLY_REQUIRE(plan->mode == FLY_MODE_F32, "the float64 light cone needs a FLY_MODE_F32 plan");
    FLY_REQUIRE(batch >= 0 && batch < (int64_t)INT32_MAX / 2, "batch out of range");
    if (batch == 0) return;
    FLY_REQUIRE(out && ldo >= batch, "bad output");
    FLY_REQUIRE(plan->n_in == 0 || (u_in && ldu >= batch), "bad input drive");
    FLY_REQUIRE(ws && ws_bytes >= fly_forward_io_f64_workspace(plan, batch), "workspace too small");
    FLY_REQUIRE(aligned(ws, 256), "workspace must be 256-byte aligned");
    hipStream_t st = as_stream(stream);
    const int32_t chunks = (int32_t)((batch + 63) / 64);
    FLY_REQUIRE(plan->max_rows * (int64_t)chunks < (int64_t)UINT32_MAX / 2, "grid too large");
    double *buf[2] = {static_cast<double *>(ws), static_cast<double *>(ws) + (size_t)plan->max_rows * batch};
    const double *prev = nullptr;
    int cur = 0;
    for (int t = 1; t <= plan->steps; ++t) {
      const int64_t nr = plan->rows_n[t];
      if (nr == 0) {
        prev = nullptr;
        continue;
      }
      hipLaunchKernelGGL(k_cone_step_f64, dim3(blocks_for(nr * chunks, 4)), dim3(256), 0, st, plan->rowptr[t].p,
                         plan->colval[t].p, plan->params[t].p, prev, batch, plan->n_in ? u_in : nullptr, ldu,
                         buf[cur], batch, (int32_t)nr, (int32_t)batch, chunks);
      check_launch("light-cone step (float64)");
      prev = buf[cur];
      cur ^= 1;
    }
    if (plan->n_out) {
      hipLaunchKernelGGL(k_outputs_f64, rows_grid(plan->n_out, batch), dim3(256), 0, st, prev, batch, plan->out_src.p,
                         plan->cbase.p, plan->n_out, batch, out, ldo);
      check_launch("outputs (float64)");
    }
  });
}

namespace fly {
namespace {

// Scratch of the literal recurrence in state type S: two (n, ld) state buffers, then the sums of split rows' pieces.
template <typename S>
size_t literal_workspace(const fly_plan &plan, int64_t batch) {
  const int64_t blk = block_cols(plan.n, sizeof(S), batch);
  return align256(2 * (size_t)plan.n * (size_t)state_ld(blk, sizeof(S)) * sizeof(S) + 256) +
         plan_pieces_bytes(plan, blk);
}

// The literal recurrence (brain.py:211-223, no-grad branch) in state type S (float32, or float16 as the reference runs
// it for float16 u): u += bias in place, then `steps` fused steps over the whole matrix, the last into h.
template <typename S>
void run_literal(const fly_plan *plan, S *u, int64_t ldu, const float *bias, int64_t batch, int32_t steps, S *h,
                 int64_t ldh, void *ws, size_t ws_bytes, hipStream_t st) {
  check_plan_device(plan);
  FLY_REQUIRE(plan->full, "the literal recurrence needs a plan from fly_plan_create_full");
  FLY_REQUIRE(steps >= 0, "negative steps");
  FLY_REQUIRE(batch >= 0 && batch < (int64_t)INT32_MAX / 2, "batch out of range");
  if (batch == 0) return;
  FLY_REQUIRE(u && bias && h && ldu >= batch && ldh >= batch, "bad argument");
  const int64_t n = plan->n;
  {
    LaunchTimer timer(FLY_K_OTHER, st);
    hipLaunchKernelGGL(k_add_bias<S>, rows_grid(n, batch), dim3(256), 0, st, u, ldu, bias, n, batch);
  }
  check_launch("bias add");
  if (steps == 0) {
    LaunchTimer timer(FLY_K_OTHER, st);
    hipLaunchKernelGGL(k_zero_rows<S>, rows_grid(n, batch), dim3(256), 0, st, h, ldh, n, batch);
    check_launch("zero state");
    return;
  }
  FLY_REQUIRE(ws && ws_bytes >= literal_workspace<S>(*plan, batch), "workspace too small");
  FLY_REQUIRE(aligned(ws, 256), "workspace must be 256-byte aligned");
  const int64_t blk = block_cols(n, sizeof(S), batch);
  float *pieces = reinterpret_cast<float *>(
      static_cast<char *>(ws) + align256(2 * (size_t)n * (size_t)state_ld(blk, sizeof(S)) * sizeof(S) + 256));
  for (int64_t c0 = 0; c0 < batch; c0 += blk) {
    const int64_t nb = std::min(blk, batch - c0);
    const int64_t lds = state_ld(nb, sizeof(S));
    S *buf[2] = {static_cast<S *>(ws), static_cast<S *>(ws) + (size_t)n * lds};
    const S *prev = nullptr;
    int cur = 0;
    for (int t = 1; t <= steps; ++t) {
      const bool last = t == steps;
      StepArgs<S, S> a{};
      a.rowptr = plan->rowptr[0].p;
      a.colval = plan->colval[0].p;
      a.params = plan->params[0].p;
      a.xprev = prev;
      a.ldx = lds;
      a.u = u + c0;
      a.ldu = ldu;
      a.xout = last ? h + c0 : buf[cur];
      a.ldo = last ? ldh : lds;
      a.out_exact = last ? 1 : 0;   // the caller's h: no store past the block's last column
      a.nrows = (int32_t)n;
      a.batch = (int32_t)nb;
      a.xbytes = prev ? buffer_bytes(n, lds, sizeof(S)) : 0;
      a.pieces = pieces;
      a.sweep_exact = std::isfinite(plan->h_max) ? 0 : 1;
      state_step(a, (double)plan->nnz[0] / (double)n, plan->tune, plan->sweep[0].get(), st);
      prev = buf[cur];
      cur ^= 1;
    }
  }
}

}  // namespace
}  // namespace fly

extern "C" size_t fly_forward_literal_workspace(const fly_plan *plan, int64_t batch) {
  return plan ? literal_workspace<float>(*plan, batch) : 0;
}

extern "C" int fly_forward_literal(const fly_plan *plan, float *u, int64_t ldu, const float *bias, int64_t batch,
                                   int32_t steps, float *h, int64_t ldh, void *ws, size_t ws_bytes, void *stream) {
  return guard([&] { run_literal<float>(plan, u, ldu, bias, batch, steps, h, ldh, ws, ws_bytes, as_stream(stream)); });
}

extern "C" size_t fly_forward_literal_f16_workspace(const fly_plan *plan, int64_t batch) {
  return plan ? literal_workspace<_Float16>(*plan, batch) : 0;
}

extern "C" int fly_forward_literal_f16(const fly_plan *plan, void *u, int64_t ldu, const float *bias, int64_t batch,
                                       int32_t steps, void *h, int64_t ldh, void *ws, size_t ws_bytes, void *stream) {
  return guard([&] {
    run_literal<_Float16>(plan, static_cast<_Float16 *>(u), ldu, bias, batch, steps, static_cast<_Float16 *>(h), ldh,
                          ws, ws_bytes, as_stream(stream));
  });
}

extern "C" size_t fly_forward_literal_f64_workspace(const fly_plan *plan, int64_t batch) {
  if (!plan) return 0;
  return 2 * (size_t)plan->n * (size_t)std::max<int64_t>(batch, 1) * sizeof(double) + 256;
}

extern "C" int fly_forward_literal_f64(const fly_plan *plan, double *u, int64_t ldu, const float *bias, int64_t batch,
                                       int32_t steps, double *h, int64_t ldh, void *ws, size_t ws_bytes, void *stream) {
  return guard([&] {
    check_plan_device(plan);
    FLY_REQUIRE(plan->full, "the literal recurrence needs a plan from fly_plan_create_full");
    FLY_REQUIRE(steps >= 0, "negative steps");
    FLY_REQUIRE(batch >= 0 && batch < (int64_t)INT32_MAX / 2, "batch out of range");
    if (batch == 0) return;
    FLY_REQUIRE(u && bias && h && ldu >= batch && ldh >= batch, "bad argument");
    const int64_t n = plan->n;
    hipStream_t st = as_stream(stream);
    hipLaunchKernelGGL(k_add_bias<double>, rows_grid(n, batch), dim3(256), 0, st, u, ldu, bias, n, batch);
    check_launch("bias add");
    if (steps == 0) {
      hipLaunchKernelGGL(k_zero_rows<double>, rows_grid(n, batch), dim3(256), 0, st, h, ldh, n, batch);
      check_launch("zero state");
      return;
    }
    FLY_REQUIRE(ws && ws_bytes >= fly_forward_literal_f64_workspace(plan, batch), "workspace too small");
    FLY_REQUIRE(aligned(ws, 256), "workspace must be 256-byte aligned");
    const int32_t chunks = (int32_t)((batch + 63) / 64);
    const int64_t waves = n * chunks;
    FLY_REQUIRE(waves < (int64_t)UINT32_MAX / 2, "grid too large");
    double *buf[2] = {static_cast<double *>(ws), static_cast<double *>(ws) + (size_t)n * batch};
    const double *prev = nullptr;
    int64_t ldp = batch;
    for (int t = 1; t <= steps; ++t) {
      const bool last = t == steps;
      double *out = last ? h : buf[(t - 1) & 1];
      const int64_t ldo = last ? ldh : batch;
      hipLaunchKernelGGL(k_literal_step_f64, dim3(blocks_for(waves, 4)), dim3(256), 0, st, plan->rowptr[0].p,
                         plan->colval[0].p, plan->params[0].p, prev, ldp, u, ldu, out, ldo, (int32_t)n, (int32_t)batch,
                         chunks);
      check_launch("literal step (float64)");
      prev = out;
      ldp = ldo;
    }
  });
}

extern "C" size_t fly_plan_step_workspace(const fly_plan *plan, int32_t t, int64_t batch) {
  if (!plan || (plan->full ? t != 1 : (t < 1 || t > plan->steps))) return 0;
  return sweep_pieces_bytes(plan->sweep[plan->full ? 0 : t].get(), batch);
}

extern "C" int fly_plan_step(const fly_plan *plan, int32_t t, const void *xprev, int64_t ldx, const void *u_in,
                             int64_t ldu, int64_t batch, void *xout, int64_t ldo, void *ws, size_t ws_bytes,
                             void *stream) {
  return guard([&] {
    check_plan_device(plan);
    FLY_REQUIRE(batch >= 0 && batch < (int64_t)INT32_MAX / 2, "batch out of range");
    FLY_REQUIRE(plan->full ? t == 1 : (t >= 1 && t <= plan->steps), "step out of range");
    const int ti = plan->full ? 0 : t;                       // the literal plan keeps its one step at index 0
    const int64_t nr = plan->rows_n[ti];
    const int64_t np = plan->full ? plan->n : plan->rows_n[t - 1];
    if (batch == 0 || nr == 0) return;
    FLY_REQUIRE(xout && ldo >= batch, "bad output state");
    FLY_REQUIRE(!xprev || ldx >= batch, "bad previous state");
    FLY_REQUIRE(plan->full || np > 0 || !xprev, "R_{t-1} is empty: the previous state must be NULL");
    FLY_REQUIRE(plan->full || np == 0 || t == 1 || xprev, "the previous state is missing");
    FLY_REQUIRE(!u_in || ldu >= batch, "bad input drive");
    const SweepTables *sweep = plan->sweep[ti].get();
    const size_t need = sweep_pieces_bytes(sweep, batch);
    FLY_REQUIRE(need == 0 || (ws && ws_bytes >= need && aligned(ws, 256)), "workspace too small or misaligned");
    // the states are caller buffers: out_exact keeps every read and write inside columns [0, batch) of a row
    hipStream_t st = as_stream(stream);
    auto run = [&](auto *xo, const auto *xp, const auto *u) {
      using S = std::remove_cv_t<std::remove_pointer_t<decltype(xo)>>;
      using U = std::remove_cv_t<std::remove_pointer_t<decltype(u)>>;
      StepArgs<S, U> a{};
      a.rowptr = plan->rowptr[ti].p;
      a.colval = plan->colval[ti].p;
      a.params = plan->params[ti].p;
      a.lead = plan->lead[ti].p;
      a.lead_flag = plan->lead_flag[ti].p;
      a.nlead = plan->nlead[ti];
      a.xprev = xp;
      a.ldx = ldx;
      a.u = u;
      a.ldu = ldu;
      a.u_padded = 0;
      a.out_exact = 1;
      a.xout = xo;
      a.ldo = ldo;
      a.nrows = (int32_t)nr;
      a.batch = (int32_t)batch;
      a.xbytes = xp ? buffer_bytes(np, ldx, sizeof(S)) : 0;
      a.pieces = static_cast<float *>(ws);
      a.sweep_exact = 1;   // caller states may hold anything
      state_step(a, nr ? (double)plan->nnz[ti] / (double)nr : 0.0, plan->tune, sweep, st);
    };
    if (plan->mode == FLY_MODE_DEVIATION_F16)
      run(static_cast<_Float16 *>(xout), static_cast<const _Float16 *>(xprev), static_cast<const _Float16 *>(u_in));
    else
      run(static_cast<float *>(xout), static_cast<const float *>(xprev), static_cast<const float *>(u_in));
  });
}

namespace fly {
namespace {

// The tuning keys: name, field and the range a value is clamped to.
struct TuningKey {
  const char *name;
  int Tuning::*field;
  int64_t lo, hi;
};
constexpr int64_t kAny = (int64_t)1 << 30;
const TuningKey kTuningKeys[] = {
    {"vec", &Tuning::vec, -kAny, kAny},
    {"unroll", &Tuning::unroll, -kAny, kAny},
    {"groups", &Tuning::groups, -kAny, kAny},
    {"rows_mode", &Tuning::rows_mode, -kAny, kAny},
    {"rows_vec", &Tuning::rows_vec, -kAny, kAny},
    {"nt_store", &Tuning::nt_store, -kAny, kAny},
    {"tiles", &Tuning::tiles, -kAny, kAny},
    {"spmm_groups", &Tuning::spmm_groups, -kAny, kAny},
    {"gemm_tile", &Tuning::gemm_tile, -kAny, kAny},
    {"download_blocks", &Tuning::download_blocks, -kAny, kAny},
    {"swept", &Tuning::swept, -1, 1},
    {"sweep_bands", &Tuning::sweep_bands, -kAny, kAny},
    {"sweep_order", &Tuning::sweep_order, -kAny, kAny},
    {"sweep_grid", &Tuning::sweep_grid, 0, 65535},
    {"sweep_piece", &Tuning::sweep_piece, 0, 1 << 20},
    {"sweep_deal", &Tuning::sweep_deal, -1, 1},
    {"sweep_paired", &Tuning::sweep_paired, -kAny, kAny},
    {"sweep_slots", &Tuning::sweep_slots, -kAny, kAny},
    {"sweep_pipe", &Tuning::sweep_pipe, -kAny, kAny},
    {"step_lds", &Tuning::step_lds, 0, 65536},
    {"nt_load", &Tuning::nt_load, -kAny, kAny},
    {"sweep_last_sync", &Tuning::sweep_last_sync, 0, 1},
};

const TuningKey &tuning_key(const char *key) {
  FLY_REQUIRE(key != nullptr, "key is null");
  for (const TuningKey &k : kTuningKeys)
    if (std::strcmp(k.name, key) == 0) return k;
  throw Error{FLY_ERR_INVALID, std::string("unknown tuning key ") + key};
}

}  // namespace
}  // namespace fly

extern "C" int fly_set_tuning(const char *key, int64_t value) {
  return guard([&] {
    const TuningKey &k = tuning_key(key);
    std::lock_guard<std::mutex> lock(g_tuning_mu);
    g_tuning.*k.field = (int)std::min(std::max(value, k.lo), k.hi);
  });
}

extern "C" int fly_get_tuning(const char *key, int64_t *value) {
  return guard([&] {
    const TuningKey &k = tuning_key(key);
    FLY_REQUIRE(value != nullptr, "value is null");
    std::lock_guard<std::mutex> lock(g_tuning_mu);
    *value = g_tuning.*k.field;
  });
}
