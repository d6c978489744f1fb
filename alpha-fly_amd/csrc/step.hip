// The recurrent state step, the hot kernel of the evaluator, and the forward_io / literal drivers.
//
// One step computes, for every row i of R_t and every board b,
//     s   = sum_e A_t[i, e] * X_{t-1}[col_e, b]                  (float32 accumulation, CSR edge order)
//     x   = clamp(s + U[usrc_i, b] + k_i, lo_i, hi_i) + e_i        (input drive only on input rows)
//     p   = prev_i >= 0 ? X_{t-1}[prev_i, b] : pdef_i
//     X_t[i, b] = lerp(p, x, a_i)
// with the state X stored (rows, ld) batch-fastest, in __half (deviation mode) or float.  This fuses the
// reference's SpMM, index_add_, gather and jiterator update (chessfly/brain.py:273-277, 310-313, 217-223)
// into one pass.
//
// Mapping: one wave64 per (row, chunk of 64*V batch columns); each lane owns V consecutive columns and
// reads them with one V*sizeof(S)-byte load per non-zero.  The row's {column, weight} pairs and its
// constants are wave-uniform and come through the scalar cache.  Non-zeros are unrolled by 8 so every lane
// keeps 8 independent gathers in flight.  Lanes past the batch re-read lane 0's address (same cache line)
// instead of branching, and only the store is masked.  Waves are numbered (tile, row, chunk-in-tile): a
// tile of batch columns is swept over all rows before the next, so the previous state's working set of one
// sweep is the tile's columns only (sized to stay in the 256 MB Infinity Cache at large batches).
#include "common.hpp"
#include "device.hpp"

namespace fly {

Tuning &tuning() {
  static Tuning t;
  return t;
}

namespace {

__device__ __forceinline__ float lerp_torch(float start, float end, float weight) {
  const bool small = fabsf(weight) < 0.5f;
  return fmaf(small ? weight : weight - 1.0f, end - start, small ? start : end);
}

// V elements of S as one vector access.  `raw` keeps a gathered vector in its storage type until the FMA
// (fp16 operands then feed v_fma_mix_f32 directly and take half the registers).
template <typename S, int V>
struct Lanes {
  typedef S vec __attribute__((ext_vector_type(V)));
  static __device__ __forceinline__ vec raw(const S *p) { return *reinterpret_cast<const vec *>(p); }
  static __device__ __forceinline__ vec zero() {
    vec v;
#pragma unroll
    for (int i = 0; i < V; ++i) v[i] = static_cast<S>(0.0f);
    return v;
  }
  static __device__ __forceinline__ float at(const vec &v, int i) { return static_cast<float>(v[i]); }
  static __device__ __forceinline__ void load(const S *p, float (&f)[V]) {
    const vec v = *reinterpret_cast<const vec *>(p);
#pragma unroll
    for (int i = 0; i < V; ++i) f[i] = static_cast<float>(v[i]);
  }
  static __device__ __forceinline__ void store(S *p, const float (&f)[V], bool nt = false) {
    vec v;
#pragma unroll
    for (int i = 0; i < V; ++i) v[i] = static_cast<S>(f[i]);
    if (nt)
      __builtin_nontemporal_store(v, reinterpret_cast<vec *>(p));
    else
      *reinterpret_cast<vec *>(p) = v;
  }
};

template <typename S>
struct Lanes<S, 1> {
  typedef S vec;
  static __device__ __forceinline__ vec raw(const S *p) { return *p; }
  static __device__ __forceinline__ vec zero() { return static_cast<S>(0.0f); }
  static __device__ __forceinline__ float at(const vec &v, int) { return static_cast<float>(v); }
  static __device__ __forceinline__ void load(const S *p, float (&f)[1]) { f[0] = static_cast<float>(*p); }
  static __device__ __forceinline__ void store(S *p, const float (&f)[1], bool nt = false) {
    if (nt)
      __builtin_nontemporal_store(static_cast<S>(f[0]), p);
    else
      *p = static_cast<S>(f[0]);
  }
};

template <typename S, typename U>
struct StepArgs {
  const int32_t *rowptr;   // |R_t| + 1, or null: no matrix term
  const int2 *colval;      // {column in X_{t-1}, float bits of the weight}
  const RowParam *params;  // |R_t|
  const S *xprev;          // X_{t-1} (rows, ldx), or null: previous state absent (zero, nothing carried)
  int64_t ldx;
  const U *u;              // input drive (n_in, ldu), or null
  int64_t ldu;
  S *xout;                 // X_t (|R_t|, ldo)
  int64_t ldo;
  int32_t nrows, batch, wpt, ntiles;
  int32_t slots;           // row slots per chunk: nrows, or ceil(nrows / G) when each wave takes G rows
  int32_t u_vec;           // the drive can be read with V-wide loads
  int32_t nt_store;        // write the new state with non-temporal stores
  uint32_t xbytes;         // bytes of X_{t-1} (rows of X_{t-1} * ldx * sizeof(S)) when below 2^31, else 0
};

// Wave -> (row, chunk of TW batch columns).  Waves are numbered (tile, row, chunk-in-tile) so a tile of
// chunks is swept over every row before the next tile starts.
struct WaveSlot {
  uint32_t row, chunk;
  bool valid;
};

template <typename S, typename U>
__device__ __forceinline__ WaveSlot wave_slot(const StepArgs<S, U> &a) {
  const uint32_t wave = blockIdx.x * 4u + (uint32_t)__builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t per_tile = (uint32_t)a.slots * (uint32_t)a.wpt;
  const uint32_t tile = wave / per_tile;
  const uint32_t in_tile = wave - tile * per_tile;
  const uint32_t row = in_tile / (uint32_t)a.wpt;
  return {row, tile * (uint32_t)a.wpt + (in_tile - row * (uint32_t)a.wpt), tile < (uint32_t)a.ntiles};
}

// A row's constants, input drive and carried state for V columns, loaded before the gathers so their
// latency overlaps the gather loop.
template <int V>
struct RowInputs {
  RowParam p;
  float u[V];
  float pv[V];
};

template <typename S, typename U, int V>
__device__ __forceinline__ void load_row_inputs(const StepArgs<S, U> &a, uint32_t row, int64_t col, bool active,
                                                RowInputs<V> &in) {
  in.p = a.params[row];
#pragma unroll
  for (int i = 0; i < V; ++i) in.u[i] = 0.0f;
  if (active && a.u != nullptr && in.p.usrc >= 0) {
    const U *src = a.u + (int64_t)in.p.usrc * a.ldu + col;
    if (a.u_vec) {
      Lanes<U, V>::load(src, in.u);
    } else {
#pragma unroll
      for (int i = 0; i < V; ++i) in.u[i] = (col + i < a.batch) ? static_cast<float>(src[i]) : 0.0f;
    }
  }
  if (active && a.xprev != nullptr && in.p.prev >= 0) {
    Lanes<S, V>::load(a.xprev + (int64_t)in.p.prev * a.ldx + col, in.pv);
  } else {
#pragma unroll
    for (int i = 0; i < V; ++i) in.pv[i] = in.p.pdef;
  }
}

// Input drive, clamp and leaky update of V columns of one row, then the store.
template <typename S, typename U, int V, bool TORCH_LERP>
__device__ __forceinline__ void finish_row(const StepArgs<S, U> &a, uint32_t row, int64_t col, const float (&acc)[V],
                                           const RowInputs<V> &in) {
  const RowParam &p = in.p;
  float out[V];
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const float x = fminf(fmaxf((acc[i] + in.u[i]) + p.k, p.lo), p.hi) + p.e;
    out[i] = TORCH_LERP ? lerp_torch(in.pv[i], x, p.a) : fmaf(p.a, x - in.pv[i], in.pv[i]);
  }
  Lanes<S, V>::store(a.xout + (int64_t)row * a.ldo + col, out, a.nt_store != 0);
}

// V elements of S at byte offset voff (per lane) + soff (wave-uniform) of a buffer: the source row's offset
// stays a scalar operand, so a gather costs the vector ALU no address arithmetic, and offsets past the end
// of the buffer read zeros instead of faulting.
template <typename S, int V>
__device__ __forceinline__ typename Lanes<S, V>::vec bload(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
  typedef typename Lanes<S, V>::vec vec;
  constexpr int kBytes = V * (int)sizeof(S);
  if constexpr (kBytes == 32) {
    typedef unsigned u4 __attribute__((ext_vector_type(4)));
    typedef unsigned u8 __attribute__((ext_vector_type(8)));
    const u4 lo = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
    const u4 hi = __builtin_amdgcn_raw_buffer_load_b128(r, voff + 16, soff, 0);
    return __builtin_bit_cast(vec, (u8)__builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
  } else if constexpr (kBytes == 16) {
    return __builtin_bit_cast(vec, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
  } else if constexpr (kBytes == 8) {
    return __builtin_bit_cast(vec, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0));
  } else if constexpr (kBytes == 4) {
    return __builtin_bit_cast(vec, __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0));
  } else {
    static_assert(kBytes == 2, "buffer gathers of 2, 4, 8, 16 or 32 bytes");
    return __builtin_bit_cast(vec, __builtin_amdgcn_raw_buffer_load_b16(r, voff, soff, 0));
  }
}


// One non-zero at a time per wave: the {column, weight} pairs are wave-uniform scalar loads, every lane
// gathers its V columns of the source row.  Chunk = 64 * V columns.
template <typename S, typename U, int V, int UNROLL, bool TORCH_LERP>
__global__ __launch_bounds__(256) void k_state_step(const StepArgs<S, U> a) {
  const WaveSlot w = wave_slot(a);
  if (!w.valid) return;
  const int lane = threadIdx.x & 63;
  const int64_t cbeg = (int64_t)w.chunk * (64 * V);
  const int64_t col = cbeg + (int64_t)lane * V;
  const bool active = col < a.batch;
  const int64_t lcol = active ? col : cbeg;

  float acc[V];
#pragma unroll
  for (int i = 0; i < V; ++i) acc[i] = 0.0f;
  RowInputs<V> in;
  load_row_inputs(a, w.row, col, active, in);

  if (a.xprev != nullptr && a.rowptr != nullptr) {
    const int32_t beg = a.rowptr[w.row], end = a.rowptr[w.row + 1];
    const S *base = a.xprev + lcol;
    int32_t e = beg;
    for (; e + UNROLL <= end; e += UNROLL) {
      int2 cv[UNROLL];
#pragma unroll
      for (int j = 0; j < UNROLL; ++j) cv[j] = a.colval[e + j];
      typename Lanes<S, V>::vec xr[UNROLL];
#pragma unroll
      for (int j = 0; j < UNROLL; ++j) xr[j] = Lanes<S, V>::raw(base + (int64_t)cv[j].x * a.ldx);
#pragma unroll
      for (int j = 0; j < UNROLL; ++j) {
        const float wt = __int_as_float(cv[j].y);
#pragma unroll
        for (int i = 0; i < V; ++i) acc[i] = fmaf(wt, Lanes<S, V>::at(xr[j], i), acc[i]);
      }
    }
    for (; e < end; ++e) {
      const int2 cv = a.colval[e];
      float xv[V];
      Lanes<S, V>::load(base + (int64_t)cv.x * a.ldx, xv);
      const float wt = __int_as_float(cv.y);
#pragma unroll
      for (int i = 0; i < V; ++i) acc[i] = fmaf(wt, xv[i], acc[i]);
    }
  }
  if (!active) return;
  finish_row<S, U, V, TORCH_LERP>(a, w.row, col, acc, in);
}


// G non-zeros at a time per wave: the wave splits into G groups of 64/G lanes, group g gathers non-zero
// e0 + j*G + g for the same chunk of (64/G) * V columns, so every load is V*sizeof(S) bytes per lane while
// the chunk (and the gather working set of a sweep) is G times narrower.  Each lane reads its group's
// {column, weight} pair with a vector load (one address per group); the pairs of the next round are loaded
// while the current round's gathers are in flight.  The G partial sums meet through cross-lane shuffles,
// and group 0 finishes the row.
template <typename S, typename U, int V, int G, int UNROLL, bool TORCH_LERP>
__global__ __launch_bounds__(256) void k_state_step_grouped(const StepArgs<S, U> a) {
  constexpr int LPG = 64 / G;
  const WaveSlot w = wave_slot(a);
  if (!w.valid) return;
  const int lane = threadIdx.x & 63;
  const int g = lane / LPG, s = lane % LPG;
  const int64_t cbeg = (int64_t)w.chunk * (LPG * V);
  const int64_t col = cbeg + (int64_t)s * V;
  const bool active = col < a.batch;
  const int64_t lcol = active ? col : cbeg;

  float acc[V];
#pragma unroll
  for (int i = 0; i < V; ++i) acc[i] = 0.0f;
  RowInputs<V> in;
  load_row_inputs(a, w.row, col, active && g == 0, in);

  if (a.xprev != nullptr && a.rowptr != nullptr) {
    const int32_t beg = a.rowptr[w.row], end = a.rowptr[w.row + 1];
    const S *base = a.xprev + lcol;
    // pairs past the row's end read as {column 0, weight 0}
    auto pairs = [&](int32_t e0, int2 (&cv)[UNROLL]) {
#pragma unroll
      for (int j = 0; j < UNROLL; ++j) {
        const int32_t e = e0 + j * G + g;
        cv[j] = e < end ? a.colval[e] : make_int2(0, 0);
      }
    };
    // With the state below 2^31 bytes a gather's address is one 24-bit multiply-add into a buffer offset
    // instead of a 64-bit product.
    const bool buf = a.xbytes != 0;
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<S *>(a.xprev), (short)0, (int)a.xbytes, kBufferWord3);
    const uint32_t row_bytes = (uint32_t)a.ldx * (uint32_t)sizeof(S), voff = (uint32_t)lcol * (uint32_t)sizeof(S);
    // The row's pairs as a buffer of (end - beg) records: pairs past the row's end read as {0, 0} with no
    // bounds test, and the round's offset is a scalar operand.
    const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int2 *>(a.colval + beg), (short)0, (end - beg) * (int)sizeof(int2), kBufferWord3);
    auto buf_pairs = [&](int32_t k, int2 (&cv)[UNROLL]) {
#pragma unroll
      for (int j = 0; j < UNROLL; ++j)
        cv[j] = __builtin_bit_cast(int2, __builtin_amdgcn_raw_buffer_load_b64(
                                             rp, (j * G + g) * (int)sizeof(int2), k * (int)sizeof(int2), 0));
    };
    int2 cv[UNROLL];
    if (beg < end) {
      if (buf)
        buf_pairs(0, cv);
      else
        pairs(beg, cv);
    }
    for (int32_t e0 = beg; e0 < end; e0 += G * UNROLL) {
      typename Lanes<S, V>::vec xr[UNROLL];
      if (buf) {
#pragma unroll
        for (int j = 0; j < UNROLL; ++j)
          xr[j] = bload<S, V>(r, (int)(__umul24((uint32_t)cv[j].x, row_bytes) + voff), 0);
      } else {
#pragma unroll
        for (int j = 0; j < UNROLL; ++j) xr[j] = Lanes<S, V>::raw(base + (int64_t)cv[j].x * a.ldx);
      }
      int2 nx[UNROLL];
      if (e0 + G * UNROLL < end) {
        if (buf)
          buf_pairs(e0 + G * UNROLL - beg, nx);
        else
          pairs(e0 + G * UNROLL, nx);
      }
#pragma unroll
      for (int j = 0; j < UNROLL; ++j) {
        const float wt = __int_as_float(cv[j].y);
#pragma unroll
        for (int i = 0; i < V; ++i) acc[i] = fmaf(wt, Lanes<S, V>::at(xr[j], i), acc[i]);
      }
#pragma unroll
      for (int j = 0; j < UNROLL; ++j) cv[j] = nx[j];
    }
#pragma unroll
    for (int i = 0; i < V; ++i) acc[i] = group_sum<LPG>(acc[i]);
  }
  if (g != 0 || !active) return;
  finish_row<S, U, V, TORCH_LERP>(a, w.row, col, acc, in);
}

// G rows at a time per wave, for steps whose rows hold few non-zeros: group g of 64/G lanes owns row
// G*slot + g and walks its non-zeros, gathering (64/G) * V columns per load; the wave loops to the longest
// of its rows with the shorter rows' loads masked off, and every group finishes its own row.
template <typename S, typename U, int V, int G, int UNROLL, bool TORCH_LERP>
__global__ __launch_bounds__(256) void k_state_step_rows(const StepArgs<S, U> a) {
  constexpr int LPG = 64 / G;
  const WaveSlot w = wave_slot(a);                // w.row counts slots of G rows
  if (!w.valid) return;
  const int lane = threadIdx.x & 63;
  const int g = lane / LPG, s = lane % LPG;
  const uint32_t row = w.row * G + g;
  const bool has_row = row < (uint32_t)a.nrows;
  const int64_t cbeg = (int64_t)w.chunk * (LPG * V);
  const int64_t col = cbeg + (int64_t)s * V;
  const bool active = has_row && col < a.batch;
  const int64_t lcol = col < a.batch ? col : cbeg;

  float acc[V];
#pragma unroll
  for (int i = 0; i < V; ++i) acc[i] = 0.0f;
  RowInputs<V> in;
  if (has_row) load_row_inputs(a, row, col, active, in);

  if (a.xprev != nullptr && a.rowptr != nullptr) {
    const int32_t beg = has_row ? a.rowptr[row] : 0, end = has_row ? a.rowptr[row + 1] : 0;
    int32_t len = end - beg;
#pragma unroll
    for (int off = LPG; off < 64; off <<= 1) len = max(len, __shfl_xor(len, off));
    const S *base = a.xprev + lcol;
    // pairs past a row's end read as {column 0, weight 0} and their gathers are skipped; the next round's
    // pairs load while this round's gathers are in flight
    auto pairs = [&](int32_t k, int2 (&cv)[UNROLL]) {
#pragma unroll
      for (int j = 0; j < UNROLL; ++j) {
        const int32_t e = beg + k + j;
        cv[j] = e < end ? a.colval[e] : make_int2(0, 0);
      }
    };
    const bool buf = a.xbytes != 0;   // 24-bit multiply-add buffer offsets, as in the grouped kernel
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<S *>(a.xprev), (short)0, (int)a.xbytes, kBufferWord3);
    const uint32_t row_bytes = (uint32_t)a.ldx * (uint32_t)sizeof(S), voff = (uint32_t)lcol * (uint32_t)sizeof(S);
    int2 cv[UNROLL];
    if (len > 0) pairs(0, cv);
    for (int32_t k = 0; k < len; k += UNROLL) {
      typename Lanes<S, V>::vec xr[UNROLL];
      if (buf) {
#pragma unroll
        for (int j = 0; j < UNROLL; ++j)
          xr[j] = (beg + k + j < end) ? bload<S, V>(r, (int)(__umul24((uint32_t)cv[j].x, row_bytes) + voff), 0)
                                      : Lanes<S, V>::zero();
      } else {
#pragma unroll
        for (int j = 0; j < UNROLL; ++j)
          xr[j] = (beg + k + j < end) ? Lanes<S, V>::raw(base + (int64_t)cv[j].x * a.ldx) : Lanes<S, V>::zero();
      }
      int2 nx[UNROLL];
      if (k + UNROLL < len) pairs(k + UNROLL, nx);
#pragma unroll
      for (int j = 0; j < UNROLL; ++j) {
        const float wt = __int_as_float(cv[j].y);
#pragma unroll
        for (int i = 0; i < V; ++i) acc[i] = fmaf(wt, Lanes<S, V>::at(xr[j], i), acc[i]);
      }
#pragma unroll
      for (int j = 0; j < UNROLL; ++j) cv[j] = nx[j];
    }
  }
  if (!active) return;
  finish_row<S, U, V, TORCH_LERP>(a, row, col, acc, in);
}


// Deviation mode (half state) updates with p + a (x - p) like the reference's fused kernel; float32 mode
// with torch.lerp's formula, like the reference's CPU path.
template <typename S, typename U, int V>
void launch_v(const StepArgs<S, U> &a, int groups, int unroll, bool rows_mode, hipStream_t st) {
  const int64_t waves = (int64_t)a.slots * a.wpt * a.ntiles;
  FLY_REQUIRE(waves < (int64_t)UINT32_MAX / 2, "state step grid too large");
  const dim3 grid(blocks_for(waves, 4)), block(256);
  LaunchTimer timer(FLY_K_STATE_STEP, st);
  constexpr bool kTL = sizeof(S) == 4;
  if constexpr (V * sizeof(S) == 32) {
    // 32-byte lanes exist for the row slots of half states only (state_step picks them for nothing else)
    hipLaunchKernelGGL((k_state_step_rows<S, U, V, 8, 4, kTL>), grid, block, 0, st, a);
    return;
  }
  if constexpr (V * sizeof(S) == 16) {
    if (rows_mode) {
      if (unroll <= 4) {   // 4 measured best for the row slots
        if (groups == 8) hipLaunchKernelGGL((k_state_step_rows<S, U, V, 8, 4, kTL>), grid, block, 0, st, a);
        else if (groups == 4) hipLaunchKernelGGL((k_state_step_rows<S, U, V, 4, 4, kTL>), grid, block, 0, st, a);
        else hipLaunchKernelGGL((k_state_step_rows<S, U, V, 2, 4, kTL>), grid, block, 0, st, a);
      } else {
        if (groups == 8) hipLaunchKernelGGL((k_state_step_rows<S, U, V, 8, 8, kTL>), grid, block, 0, st, a);
        else if (groups == 4) hipLaunchKernelGGL((k_state_step_rows<S, U, V, 4, 8, kTL>), grid, block, 0, st, a);
        else hipLaunchKernelGGL((k_state_step_rows<S, U, V, 2, 8, kTL>), grid, block, 0, st, a);
      }
      return;
    }
    if (groups == 8) {
      hipLaunchKernelGGL((k_state_step_grouped<S, U, V, 8, 4, kTL>), grid, block, 0, st, a);
      return;
    }
    if (groups == 4) {
      hipLaunchKernelGGL((k_state_step_grouped<S, U, V, 4, 8, kTL>), grid, block, 0, st, a);
      return;
    }
    if (groups == 2) {
      hipLaunchKernelGGL((k_state_step_grouped<S, U, V, 2, 8, kTL>), grid, block, 0, st, a);
      return;
    }
  }
  if (unroll >= 32)
    hipLaunchKernelGGL((k_state_step<S, U, V, 32, kTL>), grid, block, 0, st, a);
  else if (unroll >= 16)   // 8 (also for 0) measured best for one non-zero per wave
    hipLaunchKernelGGL((k_state_step<S, U, V, 16, kTL>), grid, block, 0, st, a);
  else
    hipLaunchKernelGGL((k_state_step<S, U, V, 8, kTL>), grid, block, 0, st, a);
}

template <typename S>
constexpr int max_vec() { return 16 / (int)sizeof(S); }

// Elements per lane and lane groups of the step: the tuned values when set and allowed by the alignment of
// every V-wide access, else 16-byte lanes in groups of 8 lanes, so each group gathers one 128-byte line per
// non-zero and a chunk sweep's working set is one line per source row.
template <typename S, typename U>
void pick_shape(const StepArgs<S, U> &a, int &v, int &groups) {
  auto ok = [&](int vv) {
    const size_t bytes = (size_t)vv * sizeof(S);
    if (a.ldo % vv || !aligned(a.xout, bytes)) return false;
    if (a.xprev && (a.ldx % vv || !aligned(a.xprev, bytes))) return false;
    return true;
  };
  const int want = tuning().vec;
  if (want > 0 && want <= max_vec<S>() && (want & (want - 1)) == 0 && ok(want)) {
    v = want;
  } else {
    v = 1;
    for (int vv = max_vec<S>(); vv > 1; vv >>= 1)
      if (ok(vv)) { v = vv; break; }
  }
  groups = 1;
  if (v == max_vec<S>()) {
    const int tg = tuning().groups;
    if (tg == 1 || tg == 2 || tg == 4 || tg == 8) {
      groups = tg;
    } else {
      // one 128-byte line per lane group and gather (64 half or 32 float columns), with the state's odd-line
      // row stride: measured best on MI355X for half states at B = 256-4096, and for float states 10-12% ahead
      // of 64-column chunks at B = 64-4096, light cone or not
      const int lanes = 128 / (v * (int)sizeof(S));
      groups = std::max(1, std::min(8, 64 / lanes));
    }
  }
}

template <typename S, typename U>
void state_step(StepArgs<S, U> a, double avg_nnz, hipStream_t st) {
  if (a.nrows == 0 || a.batch == 0) return;
  int v = 1, groups = 1;
  pick_shape(a, v, groups);
  // Rows shorter than 16 non-zeros on average (or no matrix at all) would leave most of a round of G
  // interleaved gathers empty: give each lane group its own row instead of its own non-zero.
  const bool rows_mode = groups > 1 && tuning().rows_mode >= 0 &&
                         (tuning().rows_mode > 0 || a.rowptr == nullptr || a.xprev == nullptr || avg_nnz < 16.0);
  // Row slots of half states read 32 bytes per lane and non-zero (two 16-byte loads, 128 columns per group):
  // a short row's wave is paced by its few dependent loads, so each round trip should carry more bytes.
  if constexpr (sizeof(S) == 2) {
    const bool wide_ok = a.ldo % 16 == 0 && aligned(a.xout, 32) && (!a.xprev || (a.ldx % 16 == 0 && aligned(a.xprev, 32)));
    if (rows_mode && v == 8 && groups == 8 && tuning().rows_vec != 8 && wide_ok) v = 16;
  }
  a.u_vec = (a.u != nullptr && a.ldu % v == 0 && aligned(a.u, (size_t)v * sizeof(U))) ? 1 : 0;
  const int width = (64 / groups) * v;
  const int chunks = (int)((a.batch + width - 1) / width);
  int tiles = tuning().tiles > 0 ? (int)tuning().tiles : chunks;
  if (tiles > chunks || chunks % tiles) tiles = chunks;
  a.ntiles = tiles;
  a.wpt = chunks / tiles;
  const int unroll = tuning().unroll > 0 ? tuning().unroll : 0;   // 0: each kernel's measured default
  a.nt_store = tuning().nt_store;
  a.slots = rows_mode ? (a.nrows + groups - 1) / groups : a.nrows;
  switch (v) {
    // only 16-byte lanes (V = 16 / sizeof(S)) have grouped and row-slot kernels, and 32-byte lanes of half
    // states a row-slot kernel; pick_shape sets groups to 1 for every other V, so rows_mode is false there too
    case 1: launch_v<S, U, 1>(a, 1, unroll, false, st); break;
    case 2: launch_v<S, U, 2>(a, 1, unroll, false, st); break;
    case 4: launch_v<S, U, 4>(a, groups, unroll, rows_mode, st); break;
    case 8:
      if constexpr (sizeof(S) == 2) launch_v<S, U, 8>(a, groups, unroll, rows_mode, st);
      break;
    default:
      if constexpr (sizeof(S) == 2) launch_v<S, U, 16>(a, groups, unroll, rows_mode, st);
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

__global__ void k_add_bias(float *__restrict__ u, int64_t ldu, const float *__restrict__ bias, int64_t n, int64_t batch) {
  const int64_t b = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (b >= batch) return;
  for (int64_t r = blockIdx.y; r < n; r += gridDim.y) u[r * ldu + b] += bias[r];
}

__global__ void k_zero_rows(float *__restrict__ h, int64_t ld, int64_t n, int64_t batch) {
  const int64_t b = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (b >= batch) return;
  for (int64_t r = blockIdx.y; r < n; r += gridDim.y) h[r * ld + b] = 0.0f;
}

}  // namespace

// Row stride of a state buffer of `elem`-byte entries: the batch rounded up to 64 columns, plus one 128-byte
// line when that leaves an even number of lines per row.  A column chunk then sits at a different line offset
// in every row, so a chunk sweep spreads over all L2 sets and channels; with a power-of-two stride it reaches a
// fraction of them (at B = 4096 the padded stride took the step from 27.3 to 23.3 ms per forward and lifted the
// L2 hit rate from 15%).
int64_t state_ld(int64_t batch, size_t elem) {
  const int64_t line = 128 / (int64_t)elem;
  int64_t ld = round_up(batch, 64);
  if ((ld / line) % 2 == 0) ld += line;
  return ld;
}

// Size of a state buffer for 32-bit buffer addressing, or 0 when it does not fit below 2^31 bytes.
uint32_t buffer_bytes(int64_t rows, int64_t ld, size_t elem) {
  const int64_t bytes = rows * ld * (int64_t)elem;
  return bytes > 0 && bytes <= (int64_t)INT32_MAX ? (uint32_t)bytes : 0u;
}

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

size_t io_workspace(const fly_plan &plan, int64_t batch) {
  const size_t es = state_bytes(plan);
  return 2 * (size_t)plan.max_rows * (size_t)state_ld(io_block(plan, batch), es) * es + 256;
}

// Runs steps 1..T of a light-cone plan.  Returns the final state (null if R_T is empty) in one of the two
// workspace buffers, whose row stride is state_ld(batch, sizeof(S)).
template <typename S, typename U>
const S *run_cone_steps(const fly_plan &plan, const U *u, int64_t ldu, int64_t batch, void *ws, hipStream_t st) {
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
    a.xprev = prev;
    a.ldx = lds;
    a.u = u;
    a.ldu = ldu;
    a.xout = buf[cur];
    a.ldo = lds;
    a.nrows = (int32_t)nr;
    a.batch = (int32_t)batch;
    a.xbytes = prev ? buffer_bytes(plan.rows_n[t - 1], lds, sizeof(S)) : 0;
    state_step(a, nr ? (double)plan.nnz[t] / (double)nr : 0.0, st);
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

template const _Float16 *run_cone_steps<_Float16, _Float16>(const fly_plan &, const _Float16 *, int64_t, int64_t, void *,
                                                            hipStream_t);
template const _Float16 *run_cone_steps<_Float16, float>(const fly_plan &, const float *, int64_t, int64_t, void *,
                                                         hipStream_t);
template const float *run_cone_steps<float, float>(const fly_plan &, const float *, int64_t, int64_t, void *, hipStream_t);

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
    for (int64_t c0 = 0; c0 < batch; c0 += blk) {
      const int64_t nb = std::min(blk, batch - c0);
      if (plan->mode == FLY_MODE_DEVIATION_F16) {
        const _Float16 *u = plan->n_in ? static_cast<const _Float16 *>(u_in) + c0 : nullptr;
        const _Float16 *fin = run_cone_steps<_Float16, _Float16>(*plan, u, ldu, nb, ws, st);
        write_outputs<_Float16>(*plan, fin, nb, out + c0, ldo, st);
      } else {
        const float *u = plan->n_in ? static_cast<const float *>(u_in) + c0 : nullptr;
        const float *fin = run_cone_steps<float, float>(*plan, u, ldu, nb, ws, st);
        write_outputs<float>(*plan, fin, nb, out + c0, ldo, st);
      }
    }
  });
}

extern "C" size_t fly_forward_literal_workspace(const fly_plan *plan, int64_t batch) {
  if (!plan) return 0;
  const int64_t blk = block_cols(plan->n, sizeof(float), batch);
  return 2 * (size_t)plan->n * (size_t)state_ld(blk, sizeof(float)) * sizeof(float) + 256;
}

extern "C" int fly_forward_literal(const fly_plan *plan, float *u, int64_t ldu, const float *bias, int64_t batch,
                                   int32_t steps, float *h, int64_t ldh, void *ws, size_t ws_bytes, void *stream) {
  return guard([&] {
    check_plan_device(plan);
    FLY_REQUIRE(plan->full, "the literal recurrence needs a plan from fly_plan_create_full");
    FLY_REQUIRE(steps >= 0, "negative steps");
    FLY_REQUIRE(batch >= 0 && batch < (int64_t)INT32_MAX / 2, "batch out of range");
    if (batch == 0) return;
    FLY_REQUIRE(u && bias && h && ldu >= batch && ldh >= batch, "bad argument");
    const int64_t n = plan->n;
    hipStream_t st = as_stream(stream);
    {
      LaunchTimer timer(FLY_K_OTHER, st);
      hipLaunchKernelGGL(k_add_bias, rows_grid(n, batch), dim3(256), 0, st, u, ldu, bias, n, batch);
    }
    check_launch("bias add");
    if (steps == 0) {
      LaunchTimer timer(FLY_K_OTHER, st);
      hipLaunchKernelGGL(k_zero_rows, rows_grid(n, batch), dim3(256), 0, st, h, ldh, n, batch);
      check_launch("zero state");
      return;
    }
    FLY_REQUIRE(ws && ws_bytes >= fly_forward_literal_workspace(plan, batch), "workspace too small");
    FLY_REQUIRE(aligned(ws, 256), "workspace must be 256-byte aligned");
    const int64_t blk = block_cols(n, sizeof(float), batch);
    for (int64_t c0 = 0; c0 < batch; c0 += blk) {
      const int64_t nb = std::min(blk, batch - c0);
      const int64_t lds = state_ld(nb, sizeof(float));
      float *buf[2] = {static_cast<float *>(ws), static_cast<float *>(ws) + (size_t)n * lds};
      const float *prev = nullptr;
      int cur = 0;
      for (int t = 1; t <= steps; ++t) {
        const bool last = t == steps;
        StepArgs<float, float> a{};
        a.rowptr = plan->rowptr[0].p;
        a.colval = plan->colval[0].p;
        a.params = plan->params[0].p;
        a.xprev = prev;
        a.ldx = lds;
        a.u = u + c0;
        a.ldu = ldu;
        a.xout = last ? h + c0 : buf[cur];
        a.ldo = last ? ldh : lds;
        a.nrows = (int32_t)n;
        a.batch = (int32_t)nb;
        a.xbytes = prev ? buffer_bytes(n, lds, sizeof(float)) : 0;
        state_step(a, (double)plan->nnz[0] / (double)n, st);
        prev = buf[cur];
        cur ^= 1;
      }
    }
  });
}

extern "C" int fly_set_tuning(const char *key, int64_t value) {
  return guard([&] {
    FLY_REQUIRE(key != nullptr, "key is null");
    const std::string k(key);
    if (k == "vec") tuning().vec = (int)value;
    else if (k == "unroll") tuning().unroll = (int)value;
    else if (k == "groups") tuning().groups = (int)value;
    else if (k == "rows_mode") tuning().rows_mode = (int)value;
    else if (k == "rows_vec") tuning().rows_vec = (int)value;
    else if (k == "nt_store") tuning().nt_store = (int)value;
    else if (k == "tiles") tuning().tiles = (int)value;
    else if (k == "spmm_groups") tuning().spmm_groups = (int)value;
    else if (k == "gemm_tile") tuning().gemm_tile = (int)value;
    else FLY_REQUIRE(false, "unknown tuning key " + k);
  });
}
