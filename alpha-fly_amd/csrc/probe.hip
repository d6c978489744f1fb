// libflyprobe.so: measurement probes for bench.py, built apart from the evaluator library.
//
// flyprobe_replay_step runs the state step's own kernels (step_kernels.hpp) built with REPLAY = 1: the same
// launch shape, wave numbering, per-row pair records and buffer-offset gathers as the evaluator's step on the
// same matrix and state layout (the banded sweep where the evaluator sweeps, over the tables that
// flyprobe_sweep_create builds with the evaluator's builder), without the arithmetic, the row inputs or the stores.  Its time is what the
// step's gather stream alone costs, which is the ceiling the fused step is measured against.
// flyprobe_replay_step_io (REPLAY = 2) adds the step's row reads (carried state, input drive, constants) and its
// stores: everything but the arithmetic of the sum.
//
// flyprobe_random_gather reads rows picked uniformly at random in the same lane layout (8 rows of 128 bytes
// per wave load, or 16 of 64 bytes), their indices streamed from memory one per read: the gather rate of a working
// set of a given size with no reuse beyond chance.  flyprobe_hashed_gather picks the rows by a hash instead, with no
// index stream: the chip's own rate of random line reads.  (Vector memory counters retire in order, so an index
// load from HBM holds up every read issued after it: the index-streamed probe measures that latency, not the
// reads.)
#include <map>
#include <mutex>
#include <string>
#include <tuple>

#include "flyprobe.h"
#include "step_kernels.hpp"

namespace fly {
namespace {

thread_local std::string g_probe_error;

// The launch-time choices of the swept kernel that a replay mirrors (flyprobe_set_tuning; fly_set_tuning's keys).
struct SweepChoice {
  int paired = 0;
  int slots = 0;
  int pipe = 0;
};
SweepChoice g_sweep;

template <typename F>
int probe_guard(F &&f) {
  try {
    f();
    return 0;
  } catch (const Error &e) {
    g_probe_error = e.msg;
  } catch (const std::exception &e) {
    g_probe_error = e.what();
  } catch (...) {
    g_probe_error = "unknown exception";
  }
  return 1;
}

__global__ void k_pack_params(const int32_t *__restrict__ prev, const int32_t *__restrict__ usrc, int64_t n,
                              RowParam *__restrict__ out) {
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i < n) out[i] = RowParam{0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, prev[i], usrc[i]};
}

__global__ void k_pack_pairs(const int32_t *__restrict__ col, const float *__restrict__ val, int64_t nnz,
                             int2 *__restrict__ out) {
  const int64_t q = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (q < nnz) out[q] = make_int2(col[q], __float_as_int(val[q]));
}

// The lead slots the evaluator's plan builds for a step matrix (build_lead_slots), kept per matrix so that repeated
// replays of one step launch without a host synchronisation after the first.
const LeadSlots &lead_slots_of(const int32_t *rowptr, int64_t nrows, int64_t nnz, hipStream_t st) {
  static std::mutex mu;
  // never destroyed: device memory is not freed from a static destructor, which may run after the HIP runtime's
  static auto *cache = new std::map<std::tuple<const int32_t *, int64_t, int64_t>, LeadSlots>();
  std::lock_guard<std::mutex> lock(mu);
  const auto key = std::make_tuple(rowptr, nrows, nnz);
  auto it = cache->find(key);
  if (it == cache->end()) {
    LeadSlots ls;
    if (nnz < 16 * nrows) ls = build_lead_slots(rowptr, nrows, nnz, st);   // the plan's rule: short rows on average
    it = cache->emplace(key, std::move(ls)).first;
  }
  return it->second;
}

// The evaluator's default shapes only (no tuning knobs): the banded sweep where the evaluator runs one (the caller
// passes the band table of flyprobe_band_table then), else lane groups of 16-byte lanes, or row slots of 16- or
// 32-byte lanes, in groups of 8 lanes with 4 rounds in flight.
template <int MODE, typename S, typename U>
void replay(StepArgs<S, U> a, int64_t nnz, const SweepTables *sweep, hipStream_t st) {
  const StepShape sh = shape_step(a, (double)nnz / (double)a.nrows, Tuning{});
  if (sweep && sh.v == 16 / (int)sizeof(S) && sh.groups == 8 && a.xbytes) {
    launch_swept<S, U, MODE>(a, *sweep, st);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) throw Error{1, std::string("replay launch: ") + hipGetErrorString(e)};
    return;
  }
  if (!(sh.rows_mode && sh.groups == 8 && a.wpt == 1 && a.lead && a.lead_flag && a.slots == (a.nrows + 7) / 8)) {
    a.lead = nullptr;   // lead slots exist for row slots of 8 rows, one chunk per tile (as the evaluator runs them)
    a.lead_flag = nullptr;
    a.nlead = 0;
  }
  const int64_t waves = (int64_t)a.slots * a.wpt * a.ntiles + (int64_t)a.nlead * a.ntiles;
  FLY_REQUIRE(waves < (int64_t)UINT32_MAX / 2, "replay grid too large");
  const dim3 grid(blocks_for(waves, 4)), block(256);
  constexpr int kV16 = 16 / (int)sizeof(S);
  FLY_REQUIRE(sh.groups == 8, "no replay for this launch shape");
  if (sh.rows_mode && sh.v == 2 * kV16) {
    if constexpr (sizeof(S) == 2)
      hipLaunchKernelGGL((k_state_step_rows<S, U, 2 * kV16, 8, 4, sizeof(S) == 4, MODE>), grid, block, 0, st, a);
  } else if (sh.rows_mode && sh.v == kV16) {
    hipLaunchKernelGGL((k_state_step_rows<S, U, kV16, 8, 4, sizeof(S) == 4, MODE>), grid, block, 0, st, a);
  } else if (!sh.rows_mode && sh.v == kV16) {
    hipLaunchKernelGGL((k_state_step_grouped<S, U, kV16, 8, 4, sizeof(S) == 4, MODE>), grid, block, 0, st, a);
  } else {
    FLY_REQUIRE(false, "no replay for this launch shape");
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) throw Error{1, std::string("replay launch: ") + hipGetErrorString(e)};
}

constexpr int kRoundsPerWave = 64;

template <int G>
__global__ __launch_bounds__(256) void k_random_gather(const char *base, uint32_t bytes, uint32_t row_bytes,
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

// Rows picked by a hash of the lane group and round, no index stream: each lane group of 64 / G lanes reads
// 128 / (G / 8) bytes of row h (16 bytes per lane), 8 reads per group in flight.  h < rows by construction, so every
// offset lies below rows * row_bytes <= bytes; the buffer resource bounds it again.
template <int G>
__global__ __launch_bounds__(256) void k_hashed_gather(const char *base, uint32_t bytes, uint32_t rows,
                                                       uint32_t row_bytes, uint32_t seed, int rounds,
                                                       float *__restrict__ sink) {
  constexpr int LPG = 64 / G;
  const int lane = threadIdx.x & 63, g = lane / LPG, s = lane % LPG;
  const uint32_t wave = blockIdx.x * 4u + (threadIdx.x >> 6);
  const __amdgpu_buffer_rsrc_t r = buffer_of(base, bytes);
  uint32_t h = (wave * (uint32_t)G + (uint32_t)g) * 2654435761u + seed;
  uint32_t fold = 0;
  typedef unsigned u4 __attribute__((ext_vector_type(4)));
  for (int k = 0; k < rounds; k += 8) {
    u4 v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      h = h * 1664525u + 1013904223u;   // a linear congruential step per read, the same in the group's lanes
      const uint32_t row = __umulhi(h, rows);
      v[j] = __builtin_amdgcn_raw_buffer_load_b128(r, (int)(row * row_bytes + (uint32_t)s * 16u), 0, 0);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) fold ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
  }
  if (fold == 0x9E3779B9u) sink[threadIdx.x] = 1.0f;   // keeps the loads alive
}

}  // namespace
}  // namespace fly

using namespace fly;

extern "C" const char *flyprobe_last_error(void) { return g_probe_error.c_str(); }

extern "C" int flyprobe_pack(const int32_t *col, const float *val, int64_t nnz, void *pairs, void *stream) {
  return probe_guard([&] {
    FLY_REQUIRE(nnz >= 0 && nnz < (int64_t)INT32_MAX, "nnz out of range");
    if (!nnz) return;
    FLY_REQUIRE(col && val && pairs && aligned(pairs, 8), "null or misaligned argument");
    hipLaunchKernelGGL(k_pack_pairs, dim3(blocks_for(nnz, 256)), dim3(256), 0, as_stream(stream), col, val, nnz,
                       static_cast<int2 *>(pairs));
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) throw Error{1, std::string("pack launch: ") + hipGetErrorString(e)};
  });
}

extern "C" int flyprobe_set_tuning(const char *key, int64_t value) {
  return probe_guard([&] {
    FLY_REQUIRE(key != nullptr, "key is null");
    const std::string k(key);
    if (k == "sweep_paired") g_sweep.paired = (int)value;
    else if (k == "sweep_slots") g_sweep.slots = (int)value;
    else if (k == "sweep_pipe") g_sweep.pipe = (int)value;
    else FLY_REQUIRE(false, "the replays mirror only sweep_paired, sweep_slots and sweep_pipe, not " + k);
  });
}

extern "C" int flyprobe_sweep_create(const int32_t *rowptr, const void *pairs, int64_t nrows, int64_t nnz,
                                     int64_t prev_rows, const int32_t *cfg, void **out, void *stream) {
  return probe_guard([&] {
    FLY_REQUIRE(rowptr && pairs && cfg && out, "null argument");
    *out = nullptr;
    FLY_REQUIRE(nrows > 0 && nrows < (int64_t)INT32_MAX / 8 && prev_rows > 0 && nnz >= 0, "size out of range");
    SweepConfig c;
    c.bands = cfg[0];
    c.paired = cfg[1];
    c.grid = cfg[2];
    c.force = cfg[3];
    c.piece = cfg[4];
    c.search = cfg[5];
    c.deal = cfg[6];
    auto t = build_sweep<int2>(rowptr, static_cast<const int2 *>(pairs), nrows, nnz, prev_rows, c, as_stream(stream));
    if (t) *out = new std::shared_ptr<const SweepTables>(std::move(t));
  });
}

extern "C" int flyprobe_sweep_destroy(void *sweep) {
  return probe_guard([&] { delete static_cast<std::shared_ptr<const SweepTables> *>(sweep); });
}

extern "C" int flyprobe_sweep_read(const void *sweep, int64_t *info, int32_t *range, int32_t *order, int32_t *split,
                                   int32_t *split_ptr, void *stream) {
  return probe_guard([&] {
    FLY_REQUIRE(sweep && info, "null argument");
    const SweepTables &t = **static_cast<const std::shared_ptr<const SweepTables> *>(sweep);
    const int64_t v[7] = {t.npos, t.pieces, t.split_rows, t.rows_per_wave, t.bands, t.grid, t.paired};
    for (int i = 0; i < 7; ++i) info[i] = v[i];
    hipStream_t st = as_stream(stream);
    auto copy = [&](int32_t *dst, const DevArray<int32_t> &src) {
      if (dst && src.n) FLY_HIP(hipMemcpyAsync(dst, src.p, sizeof(int32_t) * src.n, hipMemcpyDeviceToDevice, st));
    };
    copy(range, t.range);
    copy(order, t.order);
    copy(split, t.split);
    copy(split_ptr, t.split_ptr);
  });
}

extern "C" int flyprobe_replay_step(const int32_t *rowptr, const void *pairs, int64_t nrows, int64_t nnz,
                                    const void *xprev, int64_t prev_rows, int64_t ldx, int64_t batch, int32_t state_f16,
                                    const void *sweep, void *sink, void *stream) {
  return probe_guard([&] {
    FLY_REQUIRE(rowptr && pairs && xprev && sink, "null argument");
    const SweepTables *tables = sweep ? static_cast<const std::shared_ptr<const SweepTables> *>(sweep)->get() : nullptr;
    FLY_REQUIRE(nrows > 0 && nrows < (int64_t)INT32_MAX && nnz >= 0 && nnz < (int64_t)INT32_MAX, "size out of range");
    FLY_REQUIRE(prev_rows > 0 && batch > 0 && batch < (int64_t)INT32_MAX / 2 && ldx >= batch, "bad state layout");
    FLY_REQUIRE(aligned(sink, 256), "sink must be 256-byte aligned");
    auto run = [&](auto zero) {
      using S = decltype(zero);
      StepArgs<S, S> a{};
      a.rowptr = rowptr;
      {
        const LeadSlots &ls = lead_slots_of(rowptr, nrows, nnz, as_stream(stream));
        a.lead = ls.lead.p;
        a.lead_flag = ls.flag.p;
        a.nlead = ls.n;
      }
      a.colval = static_cast<const int2 *>(pairs);
      a.params = nullptr;
      a.xprev = static_cast<const S *>(xprev);
      a.ldx = ldx;
      a.xout = static_cast<S *>(sink);   // the sink stands in for the new state: same alignment, ldo = ldx
      a.ldo = ldx;
      a.nrows = (int32_t)nrows;
      a.batch = (int32_t)batch;
      a.xbytes = buffer_bytes(prev_rows, ldx, sizeof(S));
      a.sweep_paired = g_sweep.paired;
      a.sweep_slots = g_sweep.slots;
      a.sweep_pipe = g_sweep.pipe;
      replay<1>(a, nnz, tables, as_stream(stream));
    };
    if (state_f16)
      run(_Float16(0));
    else
      run(0.0f);
  });
}

extern "C" int flyprobe_pack_params(const int32_t *prev, const int32_t *usrc, int64_t nrows, void *params,
                                    void *stream) {
  return probe_guard([&] {
    FLY_REQUIRE(nrows >= 0 && nrows < (int64_t)INT32_MAX, "nrows out of range");
    if (!nrows) return;
    FLY_REQUIRE(prev && usrc && params && aligned(params, 16), "null or misaligned argument");
    hipLaunchKernelGGL(k_pack_params, dim3(blocks_for(nrows, 256)), dim3(256), 0, as_stream(stream), prev, usrc, nrows,
                       static_cast<RowParam *>(params));
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) throw Error{1, std::string("params launch: ") + hipGetErrorString(e)};
  });
}

extern "C" int flyprobe_replay_step_io(const int32_t *rowptr, const void *pairs, const void *params, int64_t nrows,
                                       int64_t nnz, const void *xprev, int64_t prev_rows, int64_t ldx, const float *u,
                                       int64_t n_in, int64_t ldu, void *xout, int64_t batch, int32_t state_f16,
                                       const void *sweep, void *stream) {
  return probe_guard([&] {
    FLY_REQUIRE(rowptr && pairs && params && xprev && xout, "null argument");
    const SweepTables *tables = sweep ? static_cast<const std::shared_ptr<const SweepTables> *>(sweep)->get() : nullptr;
    FLY_REQUIRE(nrows > 0 && nrows < (int64_t)INT32_MAX && nnz >= 0 && nnz < (int64_t)INT32_MAX, "size out of range");
    FLY_REQUIRE(prev_rows > 0 && batch > 0 && batch < (int64_t)INT32_MAX / 2 && ldx >= batch, "bad state layout");
    FLY_REQUIRE(!u || (n_in > 0 && ldu >= batch), "bad input drive");
    auto run = [&](auto zero) {
      using S = decltype(zero);
      StepArgs<S, float> a{};
      a.rowptr = rowptr;
      {
        const LeadSlots &ls = lead_slots_of(rowptr, nrows, nnz, as_stream(stream));
        a.lead = ls.lead.p;
        a.lead_flag = ls.flag.p;
        a.nlead = ls.n;
      }
      a.colval = static_cast<const int2 *>(pairs);
      a.params = static_cast<const RowParam *>(params);
      a.xprev = static_cast<const S *>(xprev);
      a.ldx = ldx;
      a.u = u;
      a.ldu = ldu;
      a.u_padded = 1;   // the model forward's drive: the library's padded workspace
      a.xout = static_cast<S *>(xout);
      a.ldo = ldx;
      a.nrows = (int32_t)nrows;
      a.batch = (int32_t)batch;
      a.xbytes = buffer_bytes(prev_rows, ldx, sizeof(S));
      a.sweep_paired = g_sweep.paired;
      a.sweep_slots = g_sweep.slots;
      a.sweep_pipe = g_sweep.pipe;
      replay<2>(a, nnz, tables, as_stream(stream));
    };
    if (state_f16)
      run(_Float16(0));
    else
      run(0.0f);
  });
}

extern "C" int flyprobe_hashed_gather(const void *base, int64_t bytes, int64_t rows, int64_t row_bytes,
                                      int64_t read_bytes, int64_t n, int64_t seed, float *sink, void *stream) {
  return probe_guard([&] {
    FLY_REQUIRE(base && sink, "null argument");
    FLY_REQUIRE(bytes > 0 && bytes <= INT32_MAX, "the probed buffer must hold 1 .. 2^31-1 bytes");
    FLY_REQUIRE(read_bytes == 64 || read_bytes == 128, "read_bytes must be 64 or 128");
    FLY_REQUIRE(row_bytes >= read_bytes && row_bytes < (1 << 24), "row_bytes must be read_bytes .. 2^24-1");
    FLY_REQUIRE(rows > 0 && rows * row_bytes <= bytes, "rows x row_bytes must fit the buffer");
    FLY_REQUIRE(n > 0 && n <= (int64_t)1 << 34, "n out of range");
    const int G = read_bytes == 128 ? 8 : 16;
    constexpr int kRounds = 1024;   // long-lived waves: 8,192 of them for 2^26 reads
    const int64_t waves = (n + kRounds * G - 1) / (kRounds * G);
    FLY_REQUIRE(waves < (int64_t)UINT32_MAX / 64, "probe grid too large");
    hipStream_t st = as_stream(stream);
    if (G == 8)
      hipLaunchKernelGGL(k_hashed_gather<8>, dim3(blocks_for(waves, 4)), dim3(256), 0, st,
                         static_cast<const char *>(base), (uint32_t)bytes, (uint32_t)rows, (uint32_t)row_bytes,
                         (uint32_t)seed, kRounds, sink);
    else
      hipLaunchKernelGGL(k_hashed_gather<16>, dim3(blocks_for(waves, 4)), dim3(256), 0, st,
                         static_cast<const char *>(base), (uint32_t)bytes, (uint32_t)rows, (uint32_t)row_bytes,
                         (uint32_t)seed, kRounds, sink);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) throw Error{1, std::string("gather launch: ") + hipGetErrorString(e)};
  });
}

extern "C" int flyprobe_random_gather(const void *base, int64_t bytes, int64_t row_bytes, int64_t read_bytes,
                                      const int32_t *idx, int64_t n, float *sink, void *stream) {
  return probe_guard([&] {
    FLY_REQUIRE(base && idx && sink, "null argument");
    FLY_REQUIRE(bytes > 0 && bytes <= INT32_MAX, "the probed buffer must hold 1 .. 2^31-1 bytes");
    FLY_REQUIRE(read_bytes == 64 || read_bytes == 128, "read_bytes must be 64 or 128");
    FLY_REQUIRE(row_bytes >= read_bytes && row_bytes < (1 << 24), "row_bytes must be read_bytes .. 2^24-1");
    FLY_REQUIRE(n > 0 && n <= (int64_t)1 << 34, "n out of range");
    const int G = read_bytes == 128 ? 8 : 16;
    const int64_t waves = (n + kRoundsPerWave * G - 1) / (kRoundsPerWave * G);
    FLY_REQUIRE(waves < (int64_t)UINT32_MAX, "probe grid too large");
    hipStream_t st = as_stream(stream);
    if (G == 8)
      hipLaunchKernelGGL(k_random_gather<8>, dim3(blocks_for(waves, 4)), dim3(256), 0, st,
                         static_cast<const char *>(base), (uint32_t)bytes, (uint32_t)row_bytes, idx, n, sink);
    else
      hipLaunchKernelGGL(k_random_gather<16>, dim3(blocks_for(waves, 4)), dim3(256), 0, st,
                         static_cast<const char *>(base), (uint32_t)bytes, (uint32_t)row_bytes, idx, n, sink);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) throw Error{1, std::string("gather launch: ") + hipGetErrorString(e)};
  });
}
