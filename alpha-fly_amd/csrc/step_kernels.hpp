// Device side of the recurrent state step, shared by the evaluator library and the bench's replay probe.
//
// One step computes, for every row i of R_t and every board b,
//     s   = sum_e A_t[i, e] * X_{t-1}[col_e, b]                  (float32 accumulation, CSR edge order)
//     x   = clamp(s + U[usrc_i, b] + k_i, lo_i, hi_i) + e_i        (input drive only on input rows)
//     p   = prev_i >= 0 ? X_{t-1}[prev_i, b] : pdef_i
//     X_t[i, b] = lerp(p, x, a_i)
// with the state X stored (rows, ld) batch-fastest, in __half (deviation mode) or float.
//
// Kernels: k_state_step_grouped (lane groups each gather their own non-zero of one row), k_state_step_rows
// (lane groups each own a row: steps of short rows) and k_state_step (one non-zero per wave: other lane
// widths).  Waves are numbered (tile, row, chunk-in-tile): a chunk of batch columns is swept over every row
// before the next starts, so one sweep gathers one line per source row.  REPLAY = 1 builds the gather stream
// alone, REPLAY = 2 the gathers plus the row reads and stores without the arithmetic of the sum (measurement
// builds; the evaluator library instantiates only REPLAY = 0).
#pragma once

#include "common.hpp"
#include "device.hpp"

namespace fly {

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
  int32_t u_padded;        // the drive's rows are readable up to the batch rounded up to 64 (library workspace)
  int32_t out_exact;       // caller buffers: nothing past column batch - 1 of a row may be read or written
  int32_t nt_store;        // write the new state with non-temporal stores
  uint32_t xbytes;         // bytes of X_{t-1} (rows of X_{t-1} * ldx * sizeof(S)) when below 2^31, else 0
  const int32_t *band_off; // swept steps: (nrows, bands + 1) band boundaries in colval, or null
  const int32_t *sweep_rows; // swept steps: the rows in the order the waves take them, or null (index order)
  int32_t rows_per_wave;   // swept steps: consecutive positions of that order each wave owns (set by launch_swept)
  int32_t sweep_bands;     // swept steps: bands of band_off (3 or 4)
  int32_t sweep_paired;    // swept steps: two rows per pass (1), one (-1), by the state type (0)
  int32_t sweep_slots;     // swept steps: 3 forces passes of 3 slots (0: 6 slots when a wave owns over 24 rows)
  int32_t sweep_pipe;      // swept steps: the next four rounds' gathers in flight during the sums: 0 with 3 slots,
                           // 1 also with 6, -1 never
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

// An empty asm that takes v in and out of vector registers: the compiler cannot move v's uses (a conversion, a
// select) above this point, so a value loaded before the gathers is waited for here and not before them.
template <typename T>
__device__ __forceinline__ void keep_opaque(T &v) {
  asm volatile("" : "+v"(v));
}

// A row's constants, input drive and carried state for V columns, loaded before the gathers so their latency
// overlaps the gather loop.  The drive and the carried state stay in their storage types until the epilogue
// (half the registers for float16), held opaque until then, so no wave waits for them before its gathers are
// issued.  Only lanes with a drive or a carried state load them (measured: unconditional loads of row 0 for the
// rest cost step 2, whose rows are 90% without a drive, 4% of its time).
template <typename S, typename U, int V>
struct RowInputs {
  RowParam p;
  typename Lanes<U, V>::vec u;
  typename Lanes<S, V>::vec pv;
  bool has_u, carried;
};

// The constants of each lane group's row for groups of 8 lanes: lane s reads word s of the 32-byte record and the
// group's lanes exchange them, one 4-byte load per lane instead of eight lanes each reading all 32 bytes.
template <typename S, typename U>
__device__ __forceinline__ RowParam row_param_shared8(const StepArgs<S, U> &a, uint32_t row, bool has_row, int s) {
  const int word = has_row ? reinterpret_cast<const int *>(a.params + row)[s] : 0;
  int w[8];
  static_for<8>([&](auto J) { w[decltype(J)::value] = group_bcast<8, decltype(J)::value>(word); });
  RowParam p;
  p.k = __int_as_float(w[0]);
  p.lo = __int_as_float(w[1]);
  p.hi = __int_as_float(w[2]);
  p.e = __int_as_float(w[3]);
  p.a = __int_as_float(w[4]);
  p.pdef = __int_as_float(w[5]);
  p.prev = w[6];
  p.usrc = w[7];
  return p;
}

// The drive and carried state of a row whose constants in.p are already loaded.
template <typename S, typename U, int V>
__device__ __forceinline__ void load_row_drive(const StepArgs<S, U> &a, int64_t col, bool active,
                                               RowInputs<S, U, V> &in) {
  in.has_u = active && a.u != nullptr && in.p.usrc >= 0;
  in.carried = active && a.xprev != nullptr && in.p.prev >= 0;
  in.u = Lanes<U, V>::zero();
  in.pv = Lanes<S, V>::zero();
  if (in.has_u) {
    const U *src = a.u + (int64_t)in.p.usrc * a.ldu + col;
    if (a.u_vec) {
      in.u = Lanes<U, V>::raw(src);
    } else {
      // element by element inside the batch; past it element 0 again, masked in finish_row
#pragma unroll
      for (int i = 0; i < V; ++i) {
        if constexpr (V == 1) in.u = src[0];
        else in.u[i] = src[col + i < a.batch ? i : 0];
      }
    }
  }
  if (in.carried) in.pv = Lanes<S, V>::raw(a.xprev + (int64_t)in.p.prev * a.ldx + col);
}

// The constants of a wave-uniform row, through the scalar cache: the record is read once per wave, not by every
// lane through the texture path (the params array is never written while a step runs).
template <typename S, typename U>
__device__ __forceinline__ RowParam row_param_uniform(const StepArgs<S, U> &a, uint32_t row) {
#if defined(__HIP_DEVICE_COMPILE__)
  typedef __attribute__((address_space(4))) const RowParam const_param;   // the constant address space
  return ((const_param *)a.params)[row];
#else
  return a.params[row];   // (the host pass only parses device code)
#endif
}

template <typename S, typename U, int V, bool UNIFORM = false>
__device__ __forceinline__ void load_row_inputs(const StepArgs<S, U> &a, uint32_t row, int64_t col, bool active,
                                                RowInputs<S, U, V> &in) {
  if constexpr (UNIFORM) in.p = row_param_uniform(a, row);
  else in.p = a.params[row];
  load_row_drive(a, col, active, in);
}

// Input drive, clamp and leaky update of V columns of one row, then the store.
template <typename S, typename U, int V, bool TORCH_LERP>
__device__ __forceinline__ void finish_row(const StepArgs<S, U> &a, uint32_t row, int64_t col, const float (&acc)[V],
                                           RowInputs<S, U, V> &in) {
  keep_opaque(in.u);
  keep_opaque(in.pv);
  const RowParam &p = in.p;
  float out[V];
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const float pv = in.carried ? Lanes<S, V>::at(in.pv, i) : p.pdef;
    const float u = (in.has_u && (a.u_vec || col + i < a.batch)) ? Lanes<U, V>::at(in.u, i) : 0.0f;
    const float x = fminf(fmaxf((acc[i] + u) + p.k, p.lo), p.hi) + p.e;
    out[i] = TORCH_LERP ? lerp_torch(pv, x, p.a) : fmaf(p.a, x - pv, pv);
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


// The replay of a step's memory streams (measurement builds of the kernels below): the same pair loads and
// gathers, with each gathered vector folded into a few registers by XOR instead of the FMAs, and no cross-lane
// sums.  REPLAY = 1: no row constants, input or carried state and no store; `sink` writes nothing unless the
// folded bits hit one value (so the loads stay live), into xout.  REPLAY = 2: the row reads and the store of
// the step as well, with `seed` turning the folded bits into the summed values (a denormal or zero).
template <typename S, int V>
struct ReplayBits {
  static constexpr int kWords = (V * (int)sizeof(S) + 3) / 4;
  typedef unsigned vec __attribute__((ext_vector_type(kWords)));
  static __device__ __forceinline__ vec zero() { return (vec)0u; }
  static __device__ __forceinline__ void fold(vec &bits, const typename Lanes<S, V>::vec &x, int weight) {
    if constexpr (V * sizeof(S) % 4 == 0) {
      bits ^= __builtin_bit_cast(vec, x);
    } else {
      bits[0] ^= (unsigned)__builtin_bit_cast(unsigned short, x);
    }
    bits[0] ^= (unsigned)weight;
  }
  template <typename A>
  static __device__ __forceinline__ void sink(const A &a, const vec &bits) {
    unsigned folded = 0;
#pragma unroll
    for (int i = 0; i < kWords; ++i) folded ^= bits[i];
    if (folded == 0x9E3779B9u) reinterpret_cast<unsigned *>(a.xout)[threadIdx.x] = folded;
  }
  template <int N>
  static __device__ __forceinline__ void seed(float (&acc)[N], const vec &bits) {
    acc[0] = __uint_as_float(bits[0] & 1u);
  }
};

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
  RowInputs<S, U, V> in;
  load_row_inputs<S, U, V, true>(a, w.row, col, active, in);

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
template <typename S, typename U, int V, int G, int UNROLL, bool TORCH_LERP, int REPLAY = 0>
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
  typename ReplayBits<S, V>::vec bits = ReplayBits<S, V>::zero();
  RowInputs<S, U, V> in;
  if constexpr (REPLAY != 1) load_row_inputs<S, U, V, true>(a, w.row, col, active && g == 0, in);

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
      if constexpr (REPLAY != 0) {
#pragma unroll
        for (int j = 0; j < UNROLL; ++j) ReplayBits<S, V>::fold(bits, xr[j], cv[j].y);
      } else {
#pragma unroll
        for (int j = 0; j < UNROLL; ++j) {
          const float wt = __int_as_float(cv[j].y);
#pragma unroll
          for (int i = 0; i < V; ++i) acc[i] = fmaf(wt, Lanes<S, V>::at(xr[j], i), acc[i]);
        }
      }
#pragma unroll
      for (int j = 0; j < UNROLL; ++j) cv[j] = nx[j];
    }
    if constexpr (REPLAY == 0) {
#pragma unroll
      for (int i = 0; i < V; ++i) acc[i] = group_sum<LPG>(acc[i]);
    }
  }
  if constexpr (REPLAY == 1) {
    ReplayBits<S, V>::sink(a, bits);
    return;
  }
  if constexpr (REPLAY == 2) ReplayBits<S, V>::seed(acc, bits);
  if (g != 0 || !active) return;
  finish_row<S, U, V, TORCH_LERP>(a, w.row, col, acc, in);
}

// G rows at a time per wave, for steps whose rows hold few non-zeros: group g of 64/G lanes owns row
// G*slot + g and walks its non-zeros, gathering (64/G) * V columns per load; the wave loops to the longest
// of its rows with the shorter rows' loads masked off, and every group finishes its own row.  With groups of 8
// lanes (SHARED) the group's {column, weight} records and row constants are read once per group and passed
// between its lanes (these steps are bound by the texture data path, which every per-lane copy of a record
// goes through).
template <typename S, typename U, int V, int G, int UNROLL, bool TORCH_LERP, int REPLAY = 0, bool SHARED = true>
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
  typename ReplayBits<S, V>::vec bits = ReplayBits<S, V>::zero();
  RowInputs<S, U, V> in;
  if constexpr (REPLAY != 1) {
    if constexpr (G == 8 && SHARED) {
      in.p = row_param_shared8(a, row, has_row, s);
      load_row_drive(a, col, active, in);
    } else if (has_row) {
      load_row_inputs(a, row, col, active, in);
    }
  }

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
    bool shared = false;   // the records came through the shared path below
    if constexpr (G == 8 && SHARED) {
      if (buf) {
        shared = true;
        // One 8-byte load per lane brings the group's next 8 records (lane s: record k + s of its row, the index
        // clamped into the row so every load is in bounds), and slot j of the block reaches the group's lanes by
        // a broadcast of lane j: one record load per 8 gathers instead of one per gather.  Records past a row's
        // end only feed gathers that are skipped.
        auto block = [&](int32_t k) {
          const int32_t e = max(min(beg + k + s, end - 1), 0);
          return a.colval[e];
        };
        // (the next block loads unconditionally, clamped, so no branch makes the wave drain its loads; slots past
        // a row's end gather at an offset past the buffer, which reads zeros without touching memory)
        int2 rec = len > 0 ? block(0) : make_int2(0, 0);
        for (int32_t k = 0; k < len; k += 8) {
          const int2 nxt = block(k + 8);
          static_for<8 / UNROLL>([&](auto H) {
            constexpr int h0 = decltype(H)::value * UNROLL;
            typename Lanes<S, V>::vec xr[UNROLL];
            int wj[UNROLL];
            static_for<UNROLL>([&](auto J) {
              constexpr int j = decltype(J)::value, sl = h0 + j;
              const int c = group_bcast<8, sl>(rec.x);
              wj[j] = group_bcast<8, sl>(rec.y);
              const uint32_t off = beg + k + sl < end ? __umul24((uint32_t)c, row_bytes) + voff : 0x80000000u;
              xr[j] = bload<S, V>(r, (int)off, 0);
            });
            if constexpr (REPLAY != 0) {
#pragma unroll
              for (int j = 0; j < UNROLL; ++j) ReplayBits<S, V>::fold(bits, xr[j], wj[j]);
            } else {
#pragma unroll
              for (int j = 0; j < UNROLL; ++j) {
                const float wt = __int_as_float(wj[j]);
#pragma unroll
                for (int i = 0; i < V; ++i) acc[i] = fmaf(wt, Lanes<S, V>::at(xr[j], i), acc[i]);
              }
            }
          });
          rec = nxt;
        }
      }
    }
    if (!shared) {
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
        if constexpr (REPLAY != 0) {
#pragma unroll
          for (int j = 0; j < UNROLL; ++j) ReplayBits<S, V>::fold(bits, xr[j], cv[j].y);
        } else {
#pragma unroll
          for (int j = 0; j < UNROLL; ++j) {
            const float wt = __int_as_float(cv[j].y);
#pragma unroll
            for (int i = 0; i < V; ++i) acc[i] = fmaf(wt, Lanes<S, V>::at(xr[j], i), acc[i]);
          }
        }
#pragma unroll
        for (int j = 0; j < UNROLL; ++j) cv[j] = nx[j];
      }
    }
  }
  if constexpr (REPLAY == 1) {
    ReplayBits<S, V>::sink(a, bits);
    return;
  }
  if constexpr (REPLAY == 2) ReplayBits<S, V>::seed(acc, bits);
  if (!active) return;
  finish_row<S, U, V, TORCH_LERP>(a, row, col, acc, in);
}

// ---- banded sweep of the long-row steps ---------------------------------------------------------------

constexpr int kSweepBands = 4;   // source bands of a swept step: 3 and 4 measured best (5: +3%, 6: +6% per step)

// Whether a step runs as a banded sweep: its sources overflow one XCD's 4 MB L2 at one 128-byte line per row and
// chunk (more than 32,768 rows of X_{t-1}), it has rows enough to give each of the GPU's waves several, and its
// rows are long enough for every band to hold several non-zeros.
inline bool sweep_eligible(int64_t prev_rows, int64_t rows, int64_t nnz) {
  return prev_rows > 32768 && rows >= 65536 && nnz >= 32 * rows;
}

namespace {

// Per row of A_t, where each of K bands of source rows begins among its non-zeros: band b holds the columns
// [b * prev_rows / K, (b + 1) * prev_rows / K).  off (nr, K + 1): the row's start plus the count of its columns in
// the bands before b; off[i][K] is the row's end.  A row's columns rise (CSR order of W[post, pre]), so each range
// holds exactly its band; in any other order the ranges still split the row's non-zeros between the bands.
__device__ __forceinline__ int32_t record_col(const int2 &r) { return r.x; }
__device__ __forceinline__ int32_t record_col(int32_t c) { return c; }

template <typename C>   // C: {column, weight} records (int2) or plain columns (int32_t)
__global__ void k_band_off(const int32_t *__restrict__ rowptr, const C *__restrict__ colval, int64_t nr,
                           int64_t prev_rows, int32_t K, int32_t *__restrict__ off) {
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i >= nr) return;
  const int32_t beg = rowptr[i], end = rowptr[i + 1];
  int32_t cnt[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int32_t q = beg; q < end; ++q) {
    const int64_t b = (int64_t)record_col(colval[q]) * K / prev_rows;
#pragma unroll
    for (int k = 0; k < 8; ++k) cnt[k] += (b == k) ? 1 : 0;
  }
  int32_t o = beg;
  for (int k = 0; k < K; ++k) {
    off[i * (K + 1) + k] = o;
    o += cnt[k];
  }
  off[i * (K + 1) + K] = end;
}

// The order in which the swept kernel's waves take a step's rows: each wave's own `per` consecutive rows, longest
// first (ties in index order), so the 8 rows of a slot are of like length and its rounds, which run to the longest
// of them, waste fewer gathers, while every wave keeps the same rows and share of the work.  One thread per wave's
// segment ranks each of its rows by counting the rows that go before it.
__global__ void k_sweep_order(const int32_t *__restrict__ rowptr, int64_t nr, int64_t per, int32_t *__restrict__ order) {
  const int64_t seg = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  const int64_t b = seg * per;
  if (b >= nr) return;
  const int64_t e = min(b + per, nr);
  for (int64_t i = b; i < e; ++i) {
    const int32_t li = rowptr[i + 1] - rowptr[i];
    int64_t rank = 0;
    for (int64_t j = b; j < e; ++j) {
      const int32_t lj = rowptr[j + 1] - rowptr[j];
      rank += (lj > li || (lj == li && j < i)) ? 1 : 0;
    }
    order[b + rank] = (int32_t)i;
  }
}

// Rounds one slot of a swept wave issues for one band: the longest share of its rows' band counts (a slot of
// r <= 4 rows spreads each row over 2, 4 or 8 groups, as the kernel does), padded to the 4 rounds of a gather block.
// c(i): the band count of the slot's row i.
template <typename C>
__device__ inline int slot_band_rounds(C &&c, int r) {
  const int lf = r >= 5 ? 0 : (r >= 3 ? 1 : (r == 2 ? 2 : 3));
  int m = 0;
  for (int i = 0; i < r; ++i) m = max(m, ((int)c(i) + (1 << lf) - 1) >> lf);
  return (m + 3) & ~3;
}

// Rounds one unit of a swept wave issues in band q: a slot of 8 positions, or with `paired` two slots walked as one
// pass, where each lane group walks its two rows (positions g and g + 8) back to back, so the pass runs to the
// largest pair sum, padded to 4.  c(p): the band count at position p of the unit, of which the first r hold rows.
template <typename C>
__device__ inline int unit_band_rounds(C &&c, int r, bool paired) {
  if (!paired) return slot_band_rounds(c, min(r, 8));
  int mx = 0;
  for (int g = 0; g < 8 && g < r; ++g) mx = max(mx, (int)c(g) + (g + 8 < r ? (int)c(g + 8) : 0));
  return (mx + 3) & ~3;
}

constexpr int kSearchRows = 64;     // wave segments of at most this many rows are searched (longer keep the sort)
constexpr int kSearchSteps = 200;   // moves tried per segment

// After k_sweep_order: each wave's rows rearranged between its slots so that a slot's 8 rows have like band
// counts and fewer of its rounds are padding (with `paired`, units of two slots walked as one pass).  One wave per
// segment runs a seeded local search.  At each step every lane draws two rows of the segment (xorshift32, seeded by
// segment and lane) and, if swapping them can change a unit's rounds, the change in the rounds of their units
// (summed over the bands, as unit_band_rounds counts them); the lowest change wins (ties: the lowest lane) and is
// made if it adds no rounds, so the search also walks across plateaus.  The wave keeps its rows, so its share of
// the work is unchanged.
__global__ __launch_bounds__(64) void k_sweep_order_search(const int32_t *__restrict__ band_off, int K, int64_t nr,
                                                           int64_t per, int paired, int32_t *__restrict__ order) {
  __shared__ uint16_t cnt[4][kSearchRows];
  __shared__ int32_t row[kSearchRows];
  __shared__ int32_t cost[kSearchRows / 8];   // rounds of each unit, summed over the bands
  const int lane = threadIdx.x;
  const int64_t seg = blockIdx.x;
  const int64_t b = seg * per;
  if (b >= nr || per > kSearchRows) return;
  const int m = (int)min(per, nr - b);
  for (int k = lane; k < m; k += 64) {
    const int32_t r = order[b + k];
    row[k] = r;
    for (int q = 0; q < K; ++q)
      cnt[q][k] = (uint16_t)min(band_off[(int64_t)r * (K + 1) + q + 1] - band_off[(int64_t)r * (K + 1) + q], 65535);
  }
  __syncthreads();
  const int U = paired ? 16 : 8;   // positions per unit
  const int units = (m + U - 1) / U;
  if (m <= 8) return;              // one slot: nothing to rearrange
  // rounds of unit u with the rows at positions x and y swapped (x = y = -1: as it is)
  auto unit_cost = [&](int u, int x, int y) {
    const int r = min(U, m - U * u);
    int c = 0;
    for (int q = 0; q < K; ++q)
      c += unit_band_rounds([&](int i) {
        const int p = U * u + i;
        return cnt[q][p == x ? y : (p == y ? x : p)];
      }, r, paired != 0);
    return c;
  };
  if (lane < units) cost[lane] = unit_cost(lane, -1, -1);
  __syncthreads();
  uint32_t state = (2463534242u ^ (uint32_t)(seg * 2654435761u) ^ (uint32_t)((lane + 1) * 2246822507u)) | 1u;
  auto next = [&]() {
    state ^= state << 13;
    state ^= state >> 17;
    state ^= state << 5;
    return state;
  };
  for (int step = 0; step < kSearchSteps; ++step) {
    const int i = (int)(next() % (uint32_t)m), k = (int)(next() % (uint32_t)m);
    const int ui = i / U, uk = k / U;
    int ci = 0, ck = 0, d = 1 << 20;
    if (ui != uk) {
      ci = unit_cost(ui, i, k);
      ck = unit_cost(uk, i, k);
      d = ci + ck - cost[ui] - cost[uk];
    } else if (paired && (i & 7) != (k & 7)) {   // two lane groups of one pass trade rows
      ci = ck = unit_cost(ui, i, k);
      d = ci - cost[ui];
    }
    int key = ((d + (1 << 20)) << 6) | lane;   // the lowest change, then the lowest lane
    for (int o = 32; o > 0; o >>= 1) key = min(key, __shfl_xor(key, o));
    __syncthreads();
    if ((key & 63) == lane && d <= 0) {
      const int32_t rr = row[i];
      row[i] = row[k];
      row[k] = rr;
      for (int q = 0; q < K; ++q) {
        const uint16_t cc = cnt[q][i];
        cnt[q][i] = cnt[q][k];
        cnt[q][k] = cc;
      }
      cost[ui] = ci;
      cost[uk] = ck;
    }
    __syncthreads();
  }
  for (int k = lane; k < m; k += 64) order[b + k] = row[k];
}

constexpr int kBalanceThreads = 256;
constexpr int kBalanceSteps = 600;

// After k_sweep_order_search: the rows of the 16 waves of one workgroup (one CU, whose waves meet at a barrier after
// each band) rearranged between those waves and their slots, so that each band's slowest wave is closer to the
// others.  Cost: for each band, 16 x the largest of the 16 waves' rounds (what the barrier waits for) plus their sum.
// One workgroup per group of 16 segments; at each step every thread draws two positions (xorshift32 per group and
// thread), the change in cost that swapping their rows would make is computed from the two slots' new rounds and the
// three largest wave totals of each band, and the lowest change (ties: the lowest thread) is made if it adds no cost.
// Every wave keeps its number of rows.
__global__ __launch_bounds__(kBalanceThreads) void k_sweep_order_balance(const int32_t *__restrict__ band_off, int K,
                                                                         int64_t nr, int64_t per, int paired,
                                                                         int32_t *__restrict__ order) {
  constexpr int W = 16;
  __shared__ uint16_t cnt[4][W * kSearchRows];
  __shared__ int32_t row[W * kSearchRows];
  __shared__ int32_t sr[W][kSearchRows / 8][4];   // rounds of each wave's unit (slot, or pair of slots) per band
  __shared__ int32_t tot[W][4];                   // rounds of each wave in each band
  __shared__ int32_t top[4][3][2];                // per band, the three largest wave totals (value, wave)
  __shared__ int32_t red[kBalanceThreads / 64];
  const int t = threadIdx.x;
  const int64_t grp = blockIdx.x;
  const int64_t b = grp * W * per;
  if (b >= nr || per > kSearchRows) return;
  const int P = (int)per;
  const int M = (int)min((int64_t)W * per, nr - b);
  for (int p = t; p < M; p += kBalanceThreads) {
    const int32_t r = order[b + p];
    row[p] = r;
    for (int q = 0; q < K; ++q)
      cnt[q][p] = (uint16_t)min(band_off[(int64_t)r * (K + 1) + q + 1] - band_off[(int64_t)r * (K + 1) + q], 65535);
  }
  __syncthreads();
  const int U = paired ? 16 : 8;   // positions per unit
  auto rows_of = [&](int w) { return max(0, min(P, M - w * P)); };
  // rounds of wave w's unit j in band q with the rows at positions x and y swapped (x = y = -1: as it is)
  auto rounds = [&](int w, int j, int q, int x, int y) {
    const int r = min(U, rows_of(w) - U * j);
    if (r <= 0) return 0;
    const int base = w * P + U * j;
    return unit_band_rounds([&](int i) {
      const int p = base + i;
      return cnt[q][p == x ? y : (p == y ? x : p)];
    }, r, paired != 0);
  };
  for (int x = t; x < W * (kSearchRows / 8) * 4; x += kBalanceThreads) {
    const int w = x / 32, j = (x / 4) % 8, q = x % 4;
    sr[w][j][q] = q < K ? rounds(w, j, q, -1, -1) : 0;
  }
  __syncthreads();
  if (t < W * 4) {
    int sum = 0;
    for (int j = 0; j < kSearchRows / 8; ++j) sum += sr[t / 4][j][t % 4];
    tot[t / 4][t % 4] = sum;
  }
  __syncthreads();
  auto refresh_top = [&]() {
    if (t < K) {
      int v[3] = {-1, -1, -1}, id[3] = {-1, -1, -1};
      for (int w = 0; w < W; ++w) {
        const int x = tot[w][t];
        if (x > v[0]) { v[2] = v[1]; id[2] = id[1]; v[1] = v[0]; id[1] = id[0]; v[0] = x; id[0] = w; }
        else if (x > v[1]) { v[2] = v[1]; id[2] = id[1]; v[1] = x; id[1] = w; }
        else if (x > v[2]) { v[2] = x; id[2] = w; }
      }
      for (int e = 0; e < 3; ++e) { top[t][e][0] = v[e]; top[t][e][1] = id[e]; }
    }
  };
  refresh_top();
  __syncthreads();
  uint32_t state = (2463534242u ^ (uint32_t)(grp * 2654435761u) ^ (uint32_t)((t + 1) * 2246822507u)) | 1u;
  auto next = [&]() {
    state ^= state << 13;
    state ^= state >> 17;
    state ^= state << 5;
    return state;
  };
  for (int step = 0; step < kBalanceSteps; ++step) {
    const int p1 = (int)(next() % (uint32_t)M), p2 = (int)(next() % (uint32_t)M);
    const int w1 = p1 / P, j1 = (p1 % P) / U, w2 = p2 / P, j2 = (p2 % P) / U;
    const bool same = w1 == w2 && j1 == j2;   // one unit: only two lane groups of a pass trading rows changes it
    int a1[4] = {0, 0, 0, 0}, a2[4] = {0, 0, 0, 0};
    int d = 1 << 20;
    if (!same || (paired && ((p1 % P) & 7) != ((p2 % P) & 7))) {
      d = 0;
      for (int q = 0; q < K; ++q) {
        a1[q] = rounds(w1, j1, q, p1, p2);
        a2[q] = same ? a1[q] : rounds(w2, j2, q, p1, p2);
        int t1, t2;
        if (same) {
          t1 = t2 = tot[w1][q] - sr[w1][j1][q] + a1[q];
        } else if (w1 == w2) {
          t1 = t2 = tot[w1][q] - sr[w1][j1][q] - sr[w1][j2][q] + a1[q] + a2[q];
        } else {
          t1 = tot[w1][q] - sr[w1][j1][q] + a1[q];
          t2 = tot[w2][q] - sr[w2][j2][q] + a2[q];
        }
        int other = 0;
        for (int e = 0; e < 3; ++e)
          if (top[q][e][1] != w1 && top[q][e][1] != w2) { other = max(top[q][e][0], 0); break; }
        const int newmax = max(other, max(t1, t2));
        const int dsum = w1 == w2 ? t1 - tot[w1][q] : (t1 - tot[w1][q]) + (t2 - tot[w2][q]);
        d += W * (newmax - top[q][0][0]) + dsum;
      }
    }
    int key = ((d + (1 << 20)) << 8) | t;   // the lowest change, then the lowest thread
    for (int o = 32; o > 0; o >>= 1) key = min(key, __shfl_xor(key, o));
    if ((t & 63) == 0) red[t >> 6] = key;
    __syncthreads();
    int best = red[0];
    for (int x = 1; x < kBalanceThreads / 64; ++x) best = min(best, red[x]);
    if ((best & 255) == t && d <= 0) {
      const int32_t rr = row[p1];
      row[p1] = row[p2];
      row[p2] = rr;
      for (int q = 0; q < K; ++q) {
        const uint16_t cc = cnt[q][p1];
        cnt[q][p1] = cnt[q][p2];
        cnt[q][p2] = cc;
        if (same) {
          tot[w1][q] += a1[q] - sr[w1][j1][q];
        } else if (w1 == w2) {
          tot[w1][q] += a1[q] - sr[w1][j1][q] + a2[q] - sr[w1][j2][q];
        } else {
          tot[w1][q] += a1[q] - sr[w1][j1][q];
          tot[w2][q] += a2[q] - sr[w2][j2][q];
        }
        sr[w1][j1][q] = a1[q];
        sr[w2][j2][q] = a2[q];
      }
    }
    __syncthreads();
    refresh_top();
    __syncthreads();
  }
  for (int p = t; p < M; p += kBalanceThreads) order[b + p] = row[p];
}

__global__ void k_zero_int(int32_t *p) { *p = 0; }

// The longest row of a CSR matrix (rows: nr, into *out, which starts at 0).
__global__ void k_max_row_length(const int32_t *__restrict__ rowptr, int64_t nr, int32_t *__restrict__ out) {
  int32_t m = 0;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < nr; i += (int64_t)gridDim.x * blockDim.x)
    m = max(m, rowptr[i + 1] - rowptr[i]);
  for (int off = 32; off > 0; off >>= 1) m = max(m, __shfl_xor(m, off));
  if ((threadIdx.x & 63) == 0) atomicMax(out, m);
}

}  // namespace

// Whether a step's matrix runs as a banded sweep: eligible by size, and no row much longer than the mean.  A slot's
// rounds run to the longest of its 8 rows and a workgroup's waves wait for each other after every band, so a row
// far above the mean (a hub of a graph with heavy-tailed in-degrees) would hold its whole workgroup; such a matrix
// stays on the grouped kernel.  Synchronises the stream (a plan-time decision).
inline bool sweep_suits(const int32_t *rowptr, int64_t prev_rows, int64_t nr, int64_t nnz, hipStream_t st) {
  if (!sweep_eligible(prev_rows, nr, nnz)) return false;
  DevArray<int32_t> mx(1);
  hipLaunchKernelGGL(k_zero_int, dim3(1), dim3(1), 0, st, mx.p);
  hipLaunchKernelGGL(k_max_row_length, dim3((unsigned)std::min<int64_t>(blocks_for(nr, 256), 1024)), dim3(256), 0, st,
                     rowptr, nr, mx.p);
  int32_t longest = 0;
  FLY_HIP(hipMemcpyAsync(&longest, mx.p, sizeof(longest), hipMemcpyDeviceToHost, st));
  FLY_HIP(hipStreamSynchronize(st));
  return (double)longest <= 4.0 * (double)nnz / (double)nr + 64.0;
}

// The sum over each aligned block of 2^lf lane groups of 8 lanes (lf = 0..3, wave-uniform), in every lane of the
// block: the first lf levels of group_sum's butterfly.
__device__ __forceinline__ float groups_sum(float v, int lf) {
  if (lf >= 1)
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128 /* row_ror:8 */, 0xF, 0xF, false));
  if (lf >= 2)
    v += __int_as_float(__builtin_amdgcn_permlane16_swap(__float_as_int(v), __float_as_int(v), false, false)[1]);
  if (lf >= 3)
    v += __int_as_float(__builtin_amdgcn_permlane32_swap(__float_as_int(v), __float_as_int(v), false, false)[1]);
  return v;
}

// The largest v over all lanes of the wave, as a wave-uniform value (lanes of one group of 8 hold equal values:
// the DPP rotation and the permlane swaps combine the groups as group_sum does).
__device__ __forceinline__ int wave_max_of_groups(int v) {
  v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x128 /* row_ror:8 */, 0xF, 0xF, false));
  v = max(v, (int)__builtin_amdgcn_permlane16_swap(v, v, false, false)[1]);
  v = max(v, (int)__builtin_amdgcn_permlane32_swap(v, v, false, false)[1]);
  return __builtin_amdgcn_readfirstlane(v);
}

// A long-row step as a sweep of the source rows in K bands, with each row's sums held in registers across it.
// One workgroup of 16 waves per CU, all resident at once: wave w owns rows_per_wave consecutive positions of the
// sweep order (slot j of lane group g: position w * rows_per_wave + 8 j + g, in passes of 8 * SLOTS) for every
// chunk of columns.  The order (sweep_rows, build_sweep_order) gives a slot rows of like band counts and keeps each
// band's slowest wave close to the others, while every wave keeps the same number of rows.  For each
// chunk a wave gathers band 0 of all its rows, then band 1, and so on, and the workgroup's waves meet at a barrier
// after each band: the CU's waves then draw from one band of the source rows at a time, so one XCD's L2 holds the
// lines of one band instead of the whole chunk.  (Without the barrier, issue priority lets the oldest waves run
// ahead and the working set grows.)  band_off (nrows, K + 1): row i's non-zeros of band b are
// colval[band_off[i][b] .. band_off[i][b+1]).  Lane groups of 8 lanes x 16 bytes gather one 128-byte line each; a
// slot's rounds run to the longest of the wave's 8 rows in that slot and band, the shorter rows' extra gathers from
// the row past the buffer (zeros, no memory access); a slot of 4 rows or fewer spreads each row over several lane
// groups.  PIPE keeps the next four rounds' gathers in flight during the sums.  REPLAY as for the other step
// kernels, and 3: the product alone, each row's sums stored to xout (float32 states; the training forward's A x).
template <typename S, typename U, int V, int K, int SLOTS, bool TORCH_LERP, int REPLAY = 0, bool PAIRED = false,
          bool PIPE = false>
__global__ __launch_bounds__(1024, 1) void k_state_step_swept(const StepArgs<S, U> a) {
  constexpr int UNR = 4;
  static_assert(K + 1 <= 8 && V * sizeof(S) == 16, "band starts in the lanes of a group, 16-byte lanes");
  const int lane = threadIdx.x & 63, g = lane >> 3, s = lane & 7;
  const uint32_t wave = blockIdx.x * 16u + (uint32_t)__builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t row_bytes = (uint32_t)a.ldx * (uint32_t)sizeof(S);
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<S *>(a.xprev), (short)0, (int)a.xbytes, kBufferWord3);
  const int chunks = (a.batch + 8 * V - 1) / (8 * V);
  // the rows of X_{t-1}: as a column of a record, the row just past the buffer, whose gathers read zeros (below
  // 2^24, so its 24-bit product with row_bytes is exact)
  const uint32_t past_row = a.xbytes / row_bytes;
  const int R = a.rows_per_wave;
  const uint32_t npos = (uint32_t)a.nrows;   // positions of the order: one per row
  typename ReplayBits<S, V>::vec bits = ReplayBits<S, V>::zero();
  // position p of the sweep order holds row sweep_rows[p] (p itself without an order); an entry outside the step's
  // rows reads as no row
  auto row_at = [&](uint32_t p) {
    const int32_t r = a.sweep_rows ? a.sweep_rows[p] : (int32_t)p;
    return r >= 0 && r < a.nrows ? r : -1;
  };
  for (int k0 = 0; k0 < R; k0 += 8 * SLOTS) {
    const uint32_t base = wave * (uint32_t)R + (uint32_t)k0;   // slot j, row i of the slot: position base + 8 j + i
    // Rows of slot j: a prefix of its 8 positions.  A slot of 4 rows or fewer (the last of an even split) spreads
    // each row's records over 2^lf[j] groups (lane groups g with g >> lf[j] == i take row i, each a share of every
    // band), and their sums meet before the epilogue: the slot's rounds then run to a share of its longest row
    // instead of the whole row, with the other groups idle.
    int nrow[SLOTS], lf[SLOTS];
#pragma unroll
    for (int j = 0; j < SLOTS; ++j) {
      const int64_t left = min((int64_t)R - k0 - 8 * j, (int64_t)npos - (int64_t)base - 8 * j);
      nrow[j] = (int)max<int64_t>(0, min<int64_t>(8, left));
      lf[j] = PAIRED || nrow[j] >= 5 || nrow[j] == 0 ? 0
              : (nrow[j] >= 3 ? 1 : (nrow[j] == 2 ? 2 : 3));
    }
    int off[SLOTS];   // lane s <= K: band_off[row][s]
#pragma unroll
    for (int j = 0; j < SLOTS; ++j) {
      const int i = g >> lf[j];
      const int32_t rj = i < nrow[j] ? row_at(base + 8u * j + (uint32_t)i) : -1;
      off[j] = rj >= 0 && s <= K ? a.band_off[(int64_t)rj * (K + 1) + s] : 0;
    }
    for (int c = 0; c < chunks; ++c) {
      const int64_t col = (int64_t)c * (8 * V) + (int64_t)s * V;
      const bool in_batch = col < a.batch;
      const uint32_t voff = (uint32_t)(in_batch ? col : (int64_t)c * (8 * V)) * (uint32_t)sizeof(S);
      float acc[SLOTS][V];
#pragma unroll
      for (int j = 0; j < SLOTS; ++j)
#pragma unroll
        for (int i = 0; i < V; ++i) acc[j][i] = 0.0f;
      static_for<K>([&](auto B) {
        constexpr int b = decltype(B)::value;
        if constexpr (PAIRED) {
          // Two slots' rows per pass: the group walks row A's band-b non-zeros, then row B's, so a pass runs to
          // the longest pair of the wave's 8 instead of each slot to its longest row; every gathered row feeds the
          // sums of the row it belongs to (the other row's weight is zero).
#pragma unroll
          for (int j = 0; j < SLOTS; j += 2) {
            const int bA = group_bcast<8, b>(off[j]), eA = group_bcast<8, b + 1>(off[j]);
            const int bB = group_bcast<8, b>(off[j + 1]), eB = group_bcast<8, b + 1>(off[j + 1]);
            const int nA = eA - bA, n = nA + (eB - bB);
            const int rounds = wave_max_of_groups(n);
            auto block = [&](int q0) {
              const int q = q0 + s;
              const int e = q < nA ? bA + q : (q < n ? bB + (q - nA) : (eB > bB ? eB - 1 : eA - 1));
              const int2 rc = a.colval[max(e, 0)];
              return q < n ? rc : make_int2((int)past_row, 0);   // past both rows: a gather of zeros
            };
            int2 rec = rounds > 0 ? block(0) : make_int2(0, 0);
            for (int q0 = 0; q0 < rounds; q0 += 8) {
              const int2 nxt = block(q0 + 8);
              static_for<8 / UNR>([&](auto H) {
                constexpr int h0 = decltype(H)::value * UNR;
                if (q0 + h0 < rounds) {
                  typename Lanes<S, V>::vec xr[UNR];
                  int wj[UNR];
                  static_for<UNR>([&](auto J) {
                    constexpr int u = decltype(J)::value, sl = h0 + u;
                    const int cc = group_bcast<8, sl>(rec.x);
                    wj[u] = group_bcast<8, sl>(rec.y);
                    const uint32_t o = __umul24((uint32_t)cc, row_bytes) + voff;
                    xr[u] = bload<S, V>(r, (int)o, 0);
                  });
                  if constexpr (REPLAY == 1 || REPLAY == 2) {
#pragma unroll
                    for (int u = 0; u < UNR; ++u) ReplayBits<S, V>::fold(bits, xr[u], wj[u]);
                  } else {
#pragma unroll
                    for (int u = 0; u < UNR; ++u) {
                      const float wt = __int_as_float(wj[u]);
                      const bool in_a = q0 + h0 + u < nA;
                      const float wa = in_a ? wt : 0.0f, wb = in_a ? 0.0f : wt;
#pragma unroll
                      for (int i = 0; i < V; ++i) {
                        const float x = Lanes<S, V>::at(xr[u], i);
                        acc[j][i] = fmaf(wa, x, acc[j][i]);
                        acc[j + 1][i] = fmaf(wb, x, acc[j + 1][i]);
                      }
                    }
                  }
                }
              });
              rec = nxt;
            }
          }
        } else {
#pragma unroll
        for (int j = 0; j < SLOTS; ++j) {
          int beg = group_bcast<8, b>(off[j]), end = group_bcast<8, b + 1>(off[j]);
          if (lf[j]) {   // this group's share of the row's band
            const int n = end - beg, p = g & ((1 << lf[j]) - 1), b0 = beg;
            beg = b0 + ((n * p) >> lf[j]);
            end = b0 + ((n * (p + 1)) >> lf[j]);
          }
          const int rounds = wave_max_of_groups(end - beg);
          // lane s brings record q0 + s of its row's band (clamped into the row), and round q reaches the group's
          // lanes by a broadcast of lane q; the next block of 8 loads while this one's gathers are in flight
          auto block = [&](int q0) {
            const int q = beg + q0 + s;
            const int2 rc = a.colval[max(min(q, end - 1), 0)];
            // past the row's band: the first row past the buffer (its gather reads zeros), weight 0
            return q < end ? rc : make_int2((int)past_row, 0);
          };
          if constexpr (PIPE) {
            // Four rounds' gathers stay in flight while the previous four are summed: the gathers of rounds
            // q .. q+3 are issued before the sums of rounds q-4 .. q-1 wait for theirs.
            using vec = typename Lanes<S, V>::vec;
            auto gather4 = [&](const int2 &rc, auto H, int q0, vec (&xr)[4], int (&wj)[4]) {
              constexpr int h0 = decltype(H)::value * 4;
              static_for<4>([&](auto J) {
                constexpr int u = decltype(J)::value, sl = h0 + u;
                const int cc = group_bcast<8, sl>(rc.x);
                wj[u] = group_bcast<8, sl>(rc.y);
                const uint32_t o = __umul24((uint32_t)cc, row_bytes) + voff;
                xr[u] = bload<S, V>(r, (int)o, 0);
              });
            };
            auto sum4 = [&](const vec (&xr)[4], const int (&wj)[4]) {
              if constexpr (REPLAY == 1 || REPLAY == 2) {
#pragma unroll
                for (int u = 0; u < 4; ++u) ReplayBits<S, V>::fold(bits, xr[u], wj[u]);
              } else {
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                  const float wt = __int_as_float(wj[u]);
#pragma unroll
                  for (int i = 0; i < V; ++i) acc[j][i] = fmaf(wt, Lanes<S, V>::at(xr[u], i), acc[j][i]);
                }
              }
            };
            // halves of 4 rounds: half h is lanes 4 (h % 2) .. +3 of record block h / 2; the loop body has no
            // branch, so each sum waits only for its own four gathers
            const int nh = (rounds + 3) >> 2;
            if (nh > 0) {
              vec xa[4], xb[4];
              int wa[4], wb[4];
              int2 rec = block(0);
              int2 nxt = nh > 2 ? block(8) : rec;
              gather4(rec, std::integral_constant<int, 0>{}, 0, xa, wa);
              int h = 0;
              for (; h + 2 < nh; h += 2) {   // halves h + 1 and h + 2 exist
                // the scheduler keeps this order: each sum then waits only for its own gathers
                gather4(rec, std::integral_constant<int, 1>{}, 4 * h, xb, wb);
                __builtin_amdgcn_sched_barrier(0);
                sum4(xa, wa);
                __builtin_amdgcn_sched_barrier(0);
                gather4(nxt, std::integral_constant<int, 0>{}, 4 * h + 8, xa, wa);
                rec = nxt;
                nxt = block(4 * h + 16);
                __builtin_amdgcn_sched_barrier(0);
                sum4(xb, wb);
                __builtin_amdgcn_sched_barrier(0);
              }
              if (h + 1 < nh) {
                gather4(rec, std::integral_constant<int, 1>{}, 4 * h, xb, wb);
                sum4(xa, wa);
                sum4(xb, wb);
              } else {
                sum4(xa, wa);
              }
            }
          } else {
          int2 rec = rounds > 0 ? block(0) : make_int2(0, 0);
          for (int q0 = 0; q0 < rounds; q0 += 8) {
            const int2 nxt = block(q0 + 8);
            static_for<8 / UNR>([&](auto H) {
              constexpr int h0 = decltype(H)::value * UNR;
              if (q0 + h0 < rounds) {
                typename Lanes<S, V>::vec xr[UNR];
                int wj[UNR];
                static_for<UNR>([&](auto J) {
                  constexpr int u = decltype(J)::value, sl = h0 + u;
                  const int cc = group_bcast<8, sl>(rec.x);
                  wj[u] = group_bcast<8, sl>(rec.y);
                  const uint32_t o = __umul24((uint32_t)cc, row_bytes) + voff;
                  xr[u] = bload<S, V>(r, (int)o, 0);
                });
                if constexpr (REPLAY == 1 || REPLAY == 2) {
#pragma unroll
                  for (int u = 0; u < UNR; ++u) ReplayBits<S, V>::fold(bits, xr[u], wj[u]);
                } else {
#pragma unroll
                  for (int u = 0; u < UNR; ++u) {
                    const float wt = __int_as_float(wj[u]);
#pragma unroll
                    for (int i = 0; i < V; ++i) acc[j][i] = fmaf(wt, Lanes<S, V>::at(xr[u], i), acc[j][i]);
                  }
                }
              }
            });
            rec = nxt;
          }
          }
        }
        }
        __syncthreads();   // the workgroup's waves start the next band together
      });
      if constexpr (REPLAY != 1) {
#pragma unroll
        for (int j = 0; j < SLOTS; ++j) {
          if (lf[j]) {   // the shares of a spread row meet in each of its groups
#pragma unroll
            for (int i = 0; i < V; ++i) acc[j][i] = groups_sum(acc[j][i], lf[j]);
          }
          const int i = g >> lf[j];
          const bool first = (g & ((1 << lf[j]) - 1)) == 0;
          // the position is recomputed for every chunk rather than its address kept live across the bands
          uint32_t pj = base + 8u * j + (uint32_t)i;
          asm volatile("" : "+v"(pj));
          const int32_t rs = first && i < nrow[j] && in_batch ? row_at(pj) : -1;
          if (rs >= 0) {
            const uint32_t rj = (uint32_t)rs;
            if constexpr (REPLAY == 3) {   // the product alone: y[row] = the row's sums, float32
              Lanes<S, V>::store(a.xout + (int64_t)rj * a.ldo + col, acc[j]);
            } else {
              if constexpr (REPLAY == 2) ReplayBits<S, V>::seed(acc[j], bits);
              RowInputs<S, U, V> in;
              load_row_inputs(a, rj, col, true, in);
              finish_row<S, U, V, TORCH_LERP>(a, rj, col, acc[j], in);
            }
          }
        }
      }
    }
  }
  if constexpr (REPLAY == 1) {   // keeps the loads alive; writes only if the folded bits hit one value
    unsigned folded = 0;
#pragma unroll
    for (int i = 0; i < ReplayBits<S, V>::kWords; ++i) folded ^= bits[i];
    if (folded == 0x9E3779B9u) reinterpret_cast<unsigned *>(a.xout)[threadIdx.x & 255] = folded;
  }
}

// The GPU's CU count (the swept kernel runs one workgroup per CU).
inline int cu_count() {
  static int n = -1;
  if (n < 0) {
    int dev = 0, cus = 0;
    FLY_HIP(hipGetDevice(&dev));
    FLY_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    FLY_REQUIRE(cus > 0, "no compute units");
    n = cus;
  }
  return n;
}

// The swept waves' order of a step's rows (nr, into `order`): each wave's own rows_per_wave rows, longest first
// (k_sweep_order), then rearranged between the wave's slots (k_sweep_order_search) and between the 16 waves of
// each workgroup (k_sweep_order_balance) from the band table (nr, K + 1).  `paired`: the state is float32 and the
// sweep walks two rows per pass (sweep_paired), which changes what a slot costs.
inline void build_sweep_order(const int32_t *rowptr, const int32_t *band_off, int K, int64_t nr, bool paired,
                              int32_t *order, hipStream_t st) {
  FLY_REQUIRE(nr > 0 && nr < (int64_t)INT32_MAX && (K == 3 || K == 4), "rows or bands out of range");
  const int64_t waves = 16 * (int64_t)cu_count();
  const int64_t per = (nr + waves - 1) / waves;   // launch_swept's rows_per_wave
  const int64_t segs = (nr + per - 1) / per;
  hipLaunchKernelGGL(k_sweep_order, dim3(blocks_for(segs, 64)), dim3(64), 0, st, rowptr, nr, per, order);
  if (per <= kSearchRows) {
    // the float32 kernel walks pairs of slots in one pass when a wave owns over 24 rows (launch_swept)
    const int pair = paired && K == 4 && per > 24 ? 1 : 0;
    hipLaunchKernelGGL(k_sweep_order_search, dim3((unsigned)segs), dim3(64), 0, st, band_off, K, nr, per, pair,
                       order);
    hipLaunchKernelGGL(k_sweep_order_balance, dim3((unsigned)((segs + 15) / 16)), dim3(kBalanceThreads), 0, st,
                       band_off, K, nr, per, pair, order);
  }
}

template <typename S, typename U, int K, int SLOTS, int REPLAY, bool PAIRED = false, bool PIPE = false>
void launch_swept_shape(const StepArgs<S, U> &a, unsigned grid, hipStream_t st) {
  constexpr int V = 16 / (int)sizeof(S);
  static bool fits = false;
  if (!fits) {   // the kernel's registers allow one 16-wave workgroup on every CU
    int nb = 0;
    FLY_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(
        &nb,
        reinterpret_cast<const void *>(&k_state_step_swept<S, U, V, K, SLOTS, sizeof(S) == 4, REPLAY, PAIRED, PIPE>),
        1024, 0));
    FLY_REQUIRE(nb >= 1, "the swept state step does not fit a CU");
    fits = true;
  }
  hipLaunchKernelGGL((k_state_step_swept<S, U, V, K, SLOTS, sizeof(S) == 4, REPLAY, PAIRED, PIPE>), dim3(grid),
                     dim3(1024), 0, st, a);
}

// One swept step: one workgroup per CU, the rows split evenly between the waves (one pass of up to 24 or 48 rows
// per wave; a larger step takes several passes).
template <typename S, typename U, int REPLAY>
void launch_swept(StepArgs<S, U> a, hipStream_t st) {
  const unsigned grid = (unsigned)cu_count();
  a.rows_per_wave = (int32_t)((a.nrows + 16 * (int64_t)grid - 1) / (16 * (int64_t)grid));
  const bool few = a.rows_per_wave <= 24 || a.sweep_slots == 3;
  switch (a.sweep_bands) {
    case 3:
      if (few) launch_swept_shape<S, U, 3, 3, REPLAY>(a, grid, st);
      else launch_swept_shape<S, U, 3, 6, REPLAY>(a, grid, st);
      break;
    case 4:
      // passes of 3 slots keep the next four rounds' gathers in flight during the sums (step 5 at B = 1120:
      // 1.006 -> 0.959 ms); at 6 slots the second set of gathers costs spills and gains nothing
      if (few && a.sweep_pipe >= 0) launch_swept_shape<S, U, 4, 3, REPLAY, false, true>(a, grid, st);
      else if (few) launch_swept_shape<S, U, 4, 3, REPLAY>(a, grid, st);
      else if (a.sweep_pipe > 0) launch_swept_shape<S, U, 4, 6, REPLAY, false, true>(a, grid, st);
      // float32 states walk two rows per pass (measured +1.6% at B = 1120); half states not (-5%: 16 FMAs per
      // gathered line of 8 halves cost more than the rounds they save)
      else if (a.sweep_paired > 0 || (a.sweep_paired == 0 && sizeof(S) == 4))
        launch_swept_shape<S, U, 4, 6, REPLAY, true>(a, grid, st);
      else launch_swept_shape<S, U, 4, 6, REPLAY>(a, grid, st);
      break;
    default:
      FLY_REQUIRE(false, "swept steps take 3 or 4 bands");
  }
}

template <typename S>
constexpr int max_vec() { return 16 / (int)sizeof(S); }

// Elements per lane and lane groups of the step: the tuned values when set and allowed by the alignment of
// every V-wide access, else 16-byte lanes in groups of 8 lanes, so each group gathers one 128-byte line per
// non-zero and a chunk sweep's working set is one line per source row.
template <typename S, typename U>
void pick_shape(const StepArgs<S, U> &a, const Tuning &tune, int &v, int &groups) {
  auto ok = [&](int vv) {
    const size_t bytes = (size_t)vv * sizeof(S);
    if (a.ldo % vv || !aligned(a.xout, bytes)) return false;
    // the last active lane stores vv columns: past the batch only inside the library's own padded buffers
    if (a.out_exact && a.batch % vv) return false;
    if (a.xprev && (a.ldx % vv || !aligned(a.xprev, bytes))) return false;
    return true;
  };
  const int want = tune.vec;
  if (want > 0 && want <= max_vec<S>() && (want & (want - 1)) == 0 && ok(want)) {
    v = want;
  } else {
    v = 1;
    for (int vv = max_vec<S>(); vv > 1; vv >>= 1)
      if (ok(vv)) { v = vv; break; }
  }
  groups = 1;
  if (v == max_vec<S>()) {
    const int tg = tune.groups;
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

// The launch shape of one state step, and the fields of `a` it sets (u_vec, ntiles, wpt, slots, nt_store).
struct StepShape {
  int v = 1, groups = 1, unroll = 0;
  bool rows_mode = false;
};

template <typename S, typename U>
StepShape shape_step(StepArgs<S, U> &a, double avg_nnz, const Tuning &tune) {
  StepShape sh;
  pick_shape(a, tune, sh.v, sh.groups);
  // Rows shorter than 16 non-zeros on average (or no matrix at all) would leave most of a round of G
  // interleaved gathers empty: give each lane group its own row instead of its own non-zero.
  sh.rows_mode = sh.groups > 1 && tune.rows_mode >= 0 &&
                 (tune.rows_mode > 0 || a.rowptr == nullptr || a.xprev == nullptr || avg_nnz < 16.0);
  // Row slots of half states read 32 bytes per lane and non-zero (two 16-byte loads, 128 columns per group):
  // a short row's wave is paced by its few dependent loads, so each round trip should carry more bytes.
  if constexpr (sizeof(S) == 2) {
    const bool wide_ok = a.ldo % 16 == 0 && aligned(a.xout, 32) && (!a.out_exact || a.batch % 16 == 0) &&
                         (!a.xprev || (a.ldx % 16 == 0 && aligned(a.xprev, 32)));
    if (sh.rows_mode && sh.v == 8 && sh.groups == 8 && tune.rows_vec != 8 && wide_ok) sh.v = 16;
  }
  // V-wide drive reads of the last active lane pass column batch - 1 unless the batch is a multiple of V: only
  // allowed when the drive is the library's padded workspace, never in a caller's buffer
  a.u_vec = (a.u != nullptr && a.ldu % sh.v == 0 && aligned(a.u, (size_t)sh.v * sizeof(U)) &&
             (a.u_padded || a.batch % sh.v == 0)) ? 1 : 0;
  const int width = (64 / sh.groups) * sh.v;
  const int chunks = (int)((a.batch + width - 1) / width);
  int tiles = tune.tiles > 0 ? (int)tune.tiles : chunks;
  if (tiles > chunks || chunks % tiles) tiles = chunks;
  a.ntiles = tiles;
  a.wpt = chunks / tiles;
  sh.unroll = tune.unroll > 0 ? tune.unroll : 0;   // 0: each kernel's measured default
  a.nt_store = tune.nt_store;
  a.slots = sh.rows_mode ? (a.nrows + sh.groups - 1) / sh.groups : a.nrows;
  return sh;
}

}  // namespace fly
