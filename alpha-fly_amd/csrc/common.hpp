// Shared infrastructure of the flyeval library: error capture at the C boundary, device buffers,
// small launch helpers and the per-row constant record of the state step.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <memory>
#include <string>
#include <vector>

#include "flyeval.h"

namespace fly {

struct Error {
  int code;
  std::string msg;
};

void set_error(const std::string &msg);

#define FLY_HIP(call)                                                                              \
  do {                                                                                             \
    hipError_t e_ = (call);                                                                        \
    if (e_ != hipSuccess)                                                                          \
      throw ::fly::Error{FLY_ERR_HIP, std::string(#call) + ": " + hipGetErrorString(e_)};         \
  } while (0)

#define FLY_REQUIRE(cond, msg)                                                                     \
  do {                                                                                             \
    if (!(cond)) throw ::fly::Error{FLY_ERR_INVALID, std::string(msg)};                            \
  } while (0)

// Run `f` and turn any exception into a status code plus a thread-local message.
template <typename F>
int guard(F &&f) {
  try {
    f();
    return FLY_OK;
  } catch (const Error &e) {
    set_error(e.msg);
    return e.code;
  } catch (const std::exception &e) {
    set_error(e.what());
    return FLY_ERR_INTERNAL;
  } catch (...) {
    set_error("unknown exception");
    return FLY_ERR_INTERNAL;
  }
}

inline hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }

inline void check_launch(const char *what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) throw Error{FLY_ERR_HIP, std::string(what) + " launch: " + hipGetErrorString(e)};
}

inline int current_device() {
  int d = -1;
  FLY_HIP(hipGetDevice(&d));
  return d;
}

// Device allocation owned by a library object.
template <typename T>
struct DevArray {
  T *p = nullptr;
  size_t n = 0;
  DevArray() = default;
  explicit DevArray(size_t count) { alloc(count); }
  DevArray(const DevArray &) = delete;
  DevArray &operator=(const DevArray &) = delete;
  DevArray(DevArray &&o) noexcept : p(o.p), n(o.n) { o.p = nullptr; o.n = 0; }
  DevArray &operator=(DevArray &&o) noexcept {
    if (this != &o) { release(); p = o.p; n = o.n; o.p = nullptr; o.n = 0; }
    return *this;
  }
  ~DevArray() { release(); }
  void alloc(size_t count) {
    release();
    n = count;
    if (count) FLY_HIP(hipMalloc(reinterpret_cast<void **>(&p), count * sizeof(T)));
  }
  void release() {
    if (p) (void)hipFree(p);
    p = nullptr;
    n = 0;
  }
};

inline unsigned blocks_for(int64_t work, int per_block) {
  return static_cast<unsigned>((work + per_block - 1) / per_block);
}

inline int64_t round_up(int64_t x, int64_t m) { return (x + m - 1) / m * m; }

inline bool aligned(const void *p, size_t bytes) { return (reinterpret_cast<uintptr_t>(p) % bytes) == 0; }

inline size_t align256(size_t x) { return (x + 255) / 256 * 256; }

// Row stride of a state buffer of `elem`-byte entries: the batch rounded up to 64 columns, plus one 128-byte
// line when that leaves an even number of lines per row.  A column chunk then sits at a different line offset
// in every row, so a chunk sweep spreads over all L2 sets and channels; with a power-of-two stride it reaches a
// fraction of them (at B = 4096 the padded stride took the step from 27.3 to 23.3 ms per forward and lifted the
// L2 hit rate from 15%).
inline int64_t state_ld(int64_t batch, size_t elem) {
  const int64_t line = 128 / (int64_t)elem;
  int64_t ld = round_up(batch, 64);
  if ((ld / line) % 2 == 0) ld += line;
  return ld;
}

// Size of a state buffer for 32-bit buffer addressing, or 0 when it does not fit below 2^31 bytes, a row is
// 2^24 bytes or more, or it holds 2^24 rows or more: a gather's offset is one 24-bit multiply (row index times
// row bytes), so both operands must fit 24 bits, the index of the row just past the buffer included (the swept
// step's gathers of zeros); otherwise the 64-bit path runs, or block_cols splits the batch.
inline uint32_t buffer_bytes(int64_t rows, int64_t ld, size_t elem) {
  const int64_t row_bytes = ld * (int64_t)elem;
  const int64_t bytes = rows * row_bytes;
  return bytes > 0 && bytes <= (int64_t)INT32_MAX && row_bytes < (int64_t)(1 << 24) && rows < (int64_t)(1 << 24)
             ? (uint32_t)bytes
             : 0u;
}

// Constants of one row of a state step (32 bytes, read once per row by a wave):
//   x   = clamp(s + u + k, lo, hi) + e         s = row of A_t times the previous state, u = input drive
//   p   = prev >= 0 ? state_{t-1}[prev] : pdef
//   out = lerp(p, x, a)
// Deviation mode: k = 0, lo = -k_t, hi = H - k_t, e = k_t - clamp(k_t, 0, H), pdef = 0.
// Float32 mode:   k = k_t, lo = 0, hi = H, e = 0, pdef = c_{t-1}.
struct __attribute__((aligned(16))) RowParam {
  float k, lo, hi, e, a, pdef;
  int32_t prev, usrc;
};
static_assert(sizeof(RowParam) == 32, "RowParam is 32 bytes");

// Launch timing for measurement (fly_profile_enable / fly_profile_read): a scope records a HIP event on
// the stream before and after the launches it covers, when profiling is on.
class LaunchTimer {
 public:
  LaunchTimer(int kernel_class, hipStream_t st);
  ~LaunchTimer();
  LaunchTimer(const LaunchTimer &) = delete;
  LaunchTimer &operator=(const LaunchTimer &) = delete;

 private:
  int cls_;
  hipStream_t st_;
  hipEvent_t start_ = nullptr;
};

// While one exists on a thread, LaunchTimer records nothing on that thread (and creates no events): the entry
// point that allocates nothing runs under it.
class NoLaunchEvents {
 public:
  NoLaunchEvents();
  ~NoLaunchEvents();
  NoLaunchEvents(const NoLaunchEvents &) = delete;
  NoLaunchEvents &operator=(const NoLaunchEvents &) = delete;
};

// Tuning knobs set through fly_set_tuning: the defaults that objects created afterwards capture (a plan, a dense
// plan, a fly_sweep), and that the stateless training and download entry points read at each call.
struct Tuning {
  int vec = 0;    // elements per lane of the step kernel, 0 = automatic
  int tiles = 0;  // batch tiles swept row-major, 0 = automatic
  int unroll = 0; // non-zeros gathered per wave per iteration (8, 16, 32), 0 = automatic
  int nt_store = 0;  // non-temporal stores of the new state
  int groups = 0;    // lane groups of the step (1, 2, 4, 8), each gathering its own non-zero; 0 = automatic
  int rows_mode = 0; // lane groups own rows instead of non-zeros: 1 always, -1 never, 0 for short rows
  int rows_vec = 0;  // elements per lane of row-slot steps on half states: 8 (16 bytes) or 16 (32 bytes), 0 = automatic
  int spmm_groups = 0;  // lane groups of the training SpMM on 16-byte lanes (2, 4, 8), 0 = automatic
  int gemm_tile = 0;    // dense-map workgroup tile: 1 = 64 x 64, 2 = 128 x 64, 3 = 128 x 128, 10 TM + TN, 0 = auto
  int step_lds = 0;     // bytes of LDS each state-step workgroup reserves (caps waves per SIMD), 0 = none
  int download_blocks = 0;  // workgroups of fly_evaluator_download when the call passes 0, 0 = automatic
  int swept = 0;        // long-row steps as a banded sweep: 0 automatic, -1 never, 1 any step with a matrix whatever
                        // its size (tests of small graphs)
  int sweep_bands = 0;  // source bands of a swept step (3 or 4); 0 = automatic
  int sweep_order = 0;  // swept waves take their rows in the searched order: 0 yes, -1 in the initial order
  int sweep_grid = 0;   // workgroups of a swept step; 0 = one per CU
  int sweep_piece = 0;  // split rows longer than this into pieces of at most this many non-zeros; 0 = 3 x the mean + 10
  int sweep_deal = 0;   // swept rows dealt to the waves by work: 0 where index order is unbalanced, 1 always, -1 never
  int sweep_paired = 0;  // swept waves walk two rows per pass: 1 yes, 0 or -1 one row
  int sweep_slots = 0;   // swept passes of 3 slots: 3 always, 0 when a wave owns 24 rows or fewer (else 6)
  int sweep_pipe = 0;    // swept gathers of the next four rounds in flight: 0 with 3 slots, 1 also 6, -1 never
  int nt_load = 0;       // read the carried state with non-temporal loads
  int sweep_last_sync = 0;  // 1: a swept workgroup also meets after the last band of a chunk
};
// A copy of the current defaults (taken under a lock: fly_set_tuning may run on another thread).
Tuning tuning_snapshot();

struct SweepTables;
// Sweep tables a cone has built for its steps, one entry per (step, configuration); see cone_sweep.
struct ConeSweepCache;

}  // namespace fly

// Opaque objects of the C ABI.
struct fly_cone {
  int device = -1;
  int64_t n = 0, n_edges = 0, n_in = 0, n_out = 0;
  int32_t steps = 0;
  std::vector<int64_t> rows_n;  // |R_t|, t = 0..T
  std::vector<int64_t> nnz;     // non-zeros of A_t
  std::vector<int32_t> has_op;  // A_t exists (R_{t-1} non-empty)
  std::vector<fly::DevArray<int32_t>> rows, rowptr, col, edge, prev, usrc;
  fly::DevArray<int32_t> out_src;
  fly::DevArray<int32_t> out_idx;
  // banded-sweep tables of the steps' sub-matrices: they depend on the structure only, so every plan of the cone
  // (each weight version) shares them; built on the first plan that needs them (guarded: plans of one cone may be
  // created from several threads)
  std::shared_ptr<fly::ConeSweepCache> sweep_cache;
};

struct fly_plan {
  int device = -1;
  int32_t mode = FLY_MODE_F32;
  int32_t steps = 0;
  float h_max = 10.f;
  bool full = false;  // literal recurrence plan (every row carried, u added to every row)
  int64_t n = 0, n_in = 0, n_out = 0, max_rows = 0;
  std::vector<int64_t> rows_n, nnz;
  std::vector<fly::DevArray<int32_t>> rowptr;
  std::vector<fly::DevArray<int2>> colval;  // {local column, float bits of the weight}
  std::vector<fly::DevArray<fly::RowParam>> params;
  fly::Tuning tune;   // the tuning when the plan was created: its kernels' launch choices
  // Long-row steps run as a banded sweep over their structure's tables (shared with the cone, or with the
  // fly_sweep of the whole matrix); null for the other steps.
  std::vector<std::shared_ptr<const fly::SweepTables>> sweep;
  int64_t max_pieces = 0;   // the most pieces of split rows in any swept step (their sums take workspace)
  // Steps of short rows (row slots of 8 rows): the slots holding a row far longer than the mean run first
  // (fly::build_lead_slots); empty where there are none.
  std::vector<fly::DevArray<int32_t>> lead;
  std::vector<fly::DevArray<uint8_t>> lead_flag;
  std::vector<int32_t> nlead;
  fly::DevArray<int32_t> out_src;  // position of out_idx[j] in R_T or -1
  fly::DevArray<float> cbase;      // value added to the carried state at the outputs
  fly::DevArray<float> c_out;      // c_T[out_idx]
};

// Banded-sweep tables of one CSR structure (fly_sweep_create), for the literal recurrence's whole matrix and the
// training's forward products.
struct fly_sweep {
  int device = -1;
  fly::Tuning tune;   // the tuning when it was created: the product's launch choices
  std::shared_ptr<const fly::SweepTables> t;
};
