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

#include <atomic>

#include "common.hpp"
#include "device.hpp"
#include "sweep.hpp"

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
  static __device__ __forceinline__ vec raw_nt(const S *p) {
    return __builtin_nontemporal_load(reinterpret_cast<const vec *>(p));
  }
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
  static __device__ __forceinline__ vec pack(const float (&f)[V]) {
    vec v;
#pragma unroll
    for (int i = 0; i < V; ++i) v[i] = static_cast<S>(f[i]);
    return v;
  }
  static __device__ __forceinline__ void store_raw(S *p, const vec &v, bool nt = false) {
    if (nt)
      __builtin_nontemporal_store(v, reinterpret_cast<vec *>(p));
    else
      *reinterpret_cast<vec *>(p) = v;
  }
  static __device__ __forceinline__ void store(S *p, const float (&f)[V], bool nt = false) {
    store_raw(p, pack(f), nt);
  }
};

template <typename S>
struct Lanes<S, 1> {
  typedef S vec;
  static __device__ __forceinline__ vec raw(const S *p) { return *p; }
  static __device__ __forceinline__ vec raw_nt(const S *p) { return __builtin_nontemporal_load(p); }
  static __device__ __forceinline__ vec zero() { return static_cast<S>(0.0f); }
  static __device__ __forceinline__ float at(const vec &v, int) { return static_cast<float>(v); }
  static __device__ __forceinline__ void load(const S *p, float (&f)[1]) { f[0] = static_cast<float>(*p); }
  static __device__ __forceinline__ vec pack(const float (&f)[1]) { return static_cast<S>(f[0]); }
  static __device__ __forceinline__ void store_raw(S *p, const vec &v, bool nt = false) {
    if (nt)
      __builtin_nontemporal_store(v, p);
    else
      *p = v;
  }
  static __device__ __forceinline__ void store(S *p, const float (&f)[1], bool nt = false) {
    store_raw(p, pack(f), nt);
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
  int32_t nt_load;         // read the carried state with non-temporal loads
  uint32_t xbytes;         // bytes of X_{t-1} (rows of X_{t-1} * ldx * sizeof(S)) when below 2^31, else 0
  // swept steps (set by launch_swept from the structure's SweepTables)
  const int32_t *sweep_range;  // (rows + pieces, 2 * bands) band ranges in colval
  const int32_t *sweep_order;  // (npos) the rows and pieces in the order the waves take them
  int32_t sweep_npos;          // positions of that order
  int32_t sweep_vrows;         // rows + pieces: order entries at or past it read as no row
  int32_t rows_per_wave;       // consecutive positions of the order each wave owns
  float *pieces;               // raw sums of the pieces of split rows (pieces, ldp), float32
  int64_t ldp;
  // launch-time choices of a swept step (the plan's tuning)
  int32_t sweep_paired;    // two rows per pass (1), one (-1), by the state type (0)
  int32_t sweep_slots;     // 3 forces passes of 3 slots (0: 6 slots when a wave owns over 24 rows)
  int32_t sweep_pipe;      // the next four rounds' gathers in flight during the sums: 0 with 3 slots, 1 also 6, -1 never
  int32_t sweep_exact;     // paired passes change only the owning row's sums (states that may hold inf or NaN)
  int32_t sweep_last_sync; // 1: the workgroup also meets after a chunk's last band
  // the transposed backward (swept, REPLAY == 4): each gathered line of grad_y dotted with the row's own h_{t-1}
  const float *hdot;           // (rows, ldh): h_{t-1} by row of A^T
  int64_t ldh;
  float *dots;                 // (chunks of 8 V columns, ndots): each record's dot in each chunk
  int64_t ndots;
  const int32_t *piece_row;    // (pieces): the row each piece of a split row belongs to
  int32_t accumulate;          // REPLAY 3 and 4: add the sums to xout instead of storing them
  // row slots of 8 rows: the lead slots (holding a row far longer than the mean) run first, for every chunk
  const int32_t *lead;         // (nlead) the lead slots, rising
  const uint8_t *lead_flag;    // (slots) 1 for a lead slot
  int32_t nlead;               // 0: none (and whenever the launch is not row slots of 8 rows, one chunk per tile)
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

// The row-slot kernel's waves: with lead slots, the first nlead x chunks waves take the lead slots for every chunk,
// so a slot of one very long row (a hub of a heavy-tailed in-degree) starts with the launch instead of running on
// as a tail after the rest; the chunk-major waves after them skip the lead slots.  (Needs one chunk per tile.)
template <typename S, typename U>
__device__ __forceinline__ WaveSlot rows_wave_slot(const StepArgs<S, U> &a) {
  if (a.nlead <= 0) return wave_slot(a);
  const uint32_t wave = blockIdx.x * 4u + (uint32_t)__builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t chunks = (uint32_t)a.ntiles, nl = (uint32_t)a.nlead * chunks;
  if (wave < nl) {
    const uint32_t i = wave / chunks;
    return {(uint32_t)a.lead[i], wave - i * chunks, true};
  }
  const uint32_t w2 = wave - nl, tile = w2 / (uint32_t)a.slots, slot = w2 - tile * (uint32_t)a.slots;
  const bool valid = tile < (uint32_t)a.ntiles && a.lead_flag[slot] == 0;
  return {slot, tile, valid};
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

// The constants of each lane group's row from word s of the record, held by lane s of the group: the group's lanes
// exchange the 8 words (every lane of the group must execute this).
__device__ __forceinline__ RowParam row_param_from_word(int word) {
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

// Word s of the 32-byte constants of each lane group's row, for groups of 8 lanes: lane s reads word s and the
// group's lanes exchange them (row_param_from_word), one 4-byte load per lane instead of eight lanes each reading
// all 32 bytes.  Lanes past the step's rows read row crow's word (crow: a row of the step) and drop it, so the
// load needs no branch.
template <typename S, typename U>
__device__ __forceinline__ int row_param_word(const StepArgs<S, U> &a, uint32_t crow, bool has_row, int s) {
  const int word = reinterpret_cast<const int *>(a.params + crow)[s];
  return has_row ? word : 0;
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
  if (in.carried) {
    const S *src = a.xprev + (int64_t)in.p.prev * a.ldx + col;
    in.pv = a.nt_load ? Lanes<S, V>::raw_nt(src) : Lanes<S, V>::raw(src);
  }
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
__device__ __forceinline__ void finish_value(const StepArgs<S, U> &a, int64_t col, const float (&acc)[V],
                                             RowInputs<S, U, V> &in, float (&out)[V]) {
  keep_opaque(in.u);
  keep_opaque(in.pv);
  const RowParam &p = in.p;
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const float pv = in.carried ? Lanes<S, V>::at(in.pv, i) : p.pdef;
    const float u = (in.has_u && (a.u_vec || col + i < a.batch)) ? Lanes<U, V>::at(in.u, i) : 0.0f;
    const float x = fminf(fmaxf((acc[i] + u) + p.k, p.lo), p.hi) + p.e;
    out[i] = TORCH_LERP ? lerp_torch(pv, x, p.a) : fmaf(p.a, x - pv, pv);
  }
}

template <typename S, typename U, int V, bool TORCH_LERP>
__device__ __forceinline__ void finish_row(const StepArgs<S, U> &a, uint32_t row, int64_t col, const float (&acc)[V],
                                           RowInputs<S, U, V> &in) {
  float out[V];
  finish_value<S, U, V, TORCH_LERP>(a, col, acc, in, out);
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
  const WaveSlot w = rows_wave_slot(a);           // w.row counts slots of G rows
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
  // Vector memory counters retire in order, and a load that waits on an earlier load's value costs a round trip of
  // its own: the row pointers and constants load first, together (each needs only the row; lanes past the step's
  // rows read the last row's and drop them, so neither load sits behind a branch), then the first record blocks,
  // then the drive and carried state (behind branches of their own, which may wait for them: the records are
  // already in flight then), then the gathers.
  constexpr bool kShared = G == 8 && SHARED;
  const bool mat = a.xprev != nullptr && a.rowptr != nullptr;
  const uint32_t crow = has_row ? row : (uint32_t)a.nrows - 1;
  int32_t beg = 0, end = 0;
  if (mat) {
    beg = a.rowptr[crow];
    end = a.rowptr[crow + 1];
  }
  // Shared path: the gathers need only the drive's and carried state's rows (words 7 and 6) of the constants, so
  // the other six words are passed between the group's lanes in the epilogue and hold no registers meanwhile.
  RowInputs<S, U, V> in;
  int pword = 0;
  if constexpr (REPLAY != 1) {
    if constexpr (kShared) {
      pword = row_param_word(a, crow, has_row, s);
      in.p.prev = group_bcast<8, 6>(pword);
      in.p.usrc = group_bcast<8, 7>(pword);
    } else if (has_row) {
      load_row_inputs(a, row, col, active, in);
    }
  }
  beg = has_row ? beg : 0;
  end = has_row ? end : 0;
  int32_t len = 0;
  if (mat) {
    len = end - beg;
#pragma unroll
    for (int off = LPG; off < 64; off <<= 1) len = max(len, __shfl_xor(len, off));
    len = __builtin_amdgcn_readfirstlane(len);   // the wave's longest row: equal in every lane
  }
  const bool buf = a.xbytes != 0;   // 24-bit multiply-add buffer offsets, as in the grouped kernel
  const bool shared = kShared && mat && buf;   // the records come through the shared path below
  // The shared path: one 8-byte load per lane brings the group's next 8 records (lane s: record k + s of its row,
  // the index clamped into the row so every load is in bounds), and slot j of the block reaches the group's lanes
  // by a broadcast of lane j: one record load per 8 gathers instead of one per gather.  Records past a row's end
  // only feed gathers that are skipped.
  auto block = [&](int32_t k) {
    const int32_t e = max(min(beg + k + s, end - 1), 0);
    return a.colval[e];
  };
  // The first two blocks' records load together (a row slot's rows average a few non-zeros, so most waves need one
  // or two blocks), neither behind the other's value.  Longer rows go on block by block below.
  int2 r0 = make_int2(0, 0), r1 = make_int2(0, 0);
  if (shared) {
    if (len > 0) r0 = block(0);
    if (len > 8) r1 = block(8);
  }
  if constexpr (REPLAY != 1 && kShared) load_row_drive(a, col, active, in);

  if (mat) {
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
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<S *>(a.xprev), (short)0, (int)a.xbytes, kBufferWord3);
    const uint32_t row_bytes = (uint32_t)a.ldx * (uint32_t)sizeof(S), voff = (uint32_t)lcol * (uint32_t)sizeof(S);
    if constexpr (kShared) {
      if (shared) {
        // one block of 8 rounds: the gathers and sums of records rec (lane s: record k + s of its group's row), in
        // steps of UNROLL rounds up to the wave's longest row (len is wave-uniform)
        auto run = [&](const int2 rec, int32_t k) {
          static_for<8 / UNROLL>([&](auto H) {
            constexpr int h0 = decltype(H)::value * UNROLL;
            if (h0 > 0 && k + h0 >= len) return;
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
        };
        // Rows past two blocks go on block by block, the next one's load in flight (it loads unconditionally,
        // clamped, so no branch makes the wave drain its loads; slots past a row's end gather at an offset past
        // the buffer, which reads zeros without touching memory).
        if (len > 0) run(r0, 0);
        if (len > 8) run(r1, 8);
        if (len > 16) {
          int2 rec = block(16);
          for (int32_t k = 16; k < len; k += 8) {
            const int2 nxt = block(k + 8);
            run(rec, k);
            rec = nxt;
          }
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
  if constexpr (kShared) {   // every lane of the group takes part in the exchange
    keep_opaque(pword);
    in.p = row_param_from_word(pword);
  }
  if (!active) return;
  finish_row<S, U, V, TORCH_LERP>(a, row, col, acc, in);
}

// ---- banded sweep of the long-row steps ---------------------------------------------------------------

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
// chunk of columns.  The order (SweepTables, build_sweep) gives a slot rows of like band counts and keeps each
// band's slowest wave close to the others, while every wave keeps the same number of rows.  A position holds a row
// of the step, or a piece of a row the tables split (rows far longer than the mean): a piece stores its raw sums to
// `pieces`, and k_sweep_finish adds a split row's pieces and runs its epilogue.  For each
// chunk a wave gathers band 0 of all its rows, then band 1, and so on, and the workgroup's waves meet at a barrier
// after each band: the CU's waves then draw from one band of the source rows at a time, so one XCD's L2 holds the
// lines of one band instead of the whole chunk.  (Without the barrier, issue priority lets the oldest waves run
// ahead and the working set grows.)  sweep_range (rows + pieces, 2K): row or piece v's non-zeros of band b are
// colval[range[v][2b] .. range[v][2b+1]).  Lane groups of 8 lanes x 16 bytes gather one 128-byte line each; a
// slot's rounds run to the longest of the wave's 8 rows in that slot and band, the shorter rows' extra gathers from
// the row past the buffer (zeros, no memory access); a slot of 4 rows or fewer spreads each row over several lane
// groups.  PAIRED walks two slots' rows per pass (1: the other row's weight is zero, for states that hold no inf
// or NaN; 2: only the owning row's sums change).  PIPE keeps the next four rounds' gathers in flight during the
// sums.  Vector memory counters retire in order, so every load is placed where waiting for it costs nothing extra:
// a slot's first record blocks load together, the next band's first records load with a band's last slot, and the
// epilogue stores a batch's new states after the next batch's row reads.  REPLAY as for the other step kernels, and 3: the product alone, each row's sums stored to xout (float32
// states; the training forward's A x); 4: the training backward's pass over A^T, the product grad_h = A^T grad_y
// added to xout and, per record and chunk, the dot of the gathered line of grad_y with the row's own h_{t-1}
// (hdot) stored to dots (dL/dw's share of the chunk).
template <typename S, typename U, int V, int K, int SLOTS, bool TORCH_LERP, int REPLAY = 0, int PAIRED = 0,
          bool PIPE = false>
__global__ __launch_bounds__(1024, 1) void k_state_step_swept(const StepArgs<S, U> a) {
  constexpr int UNR = 4;
  static_assert(2 * K <= 8 && V * sizeof(S) == 16, "band ranges in the lanes of a group, 16-byte lanes");
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
  const uint32_t npos = (uint32_t)a.sweep_npos;   // positions of the order
  typename ReplayBits<S, V>::vec bits = ReplayBits<S, V>::zero();
  // Per wave, slot and lane: the row the lane's group finishes in the epilogue (-1: none) and word s of that row's
  // 32-byte constants, written once per pass and read by the same lane after every chunk, so the epilogue issues
  // the loads of several rows' carried state and drive at once instead of three dependent loads per row.
  const int wv = threadIdx.x >> 6;
  __shared__ int ep_row[REPLAY != 1 ? 16 * SLOTS * 64 : 1];
  __shared__ int ep_par[REPLAY == 0 || REPLAY == 2 ? 16 * SLOTS * 64 : 1];
  // position p of the sweep order holds row (or nrows + piece) sweep_order[p]; an entry outside the step's rows and
  // pieces reads as no row
  auto row_at = [&](uint32_t p) {
    const int32_t r = a.sweep_order[p];
    return r >= 0 && r < a.sweep_vrows ? r : -1;
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
      lf[j] = PAIRED != 0 || nrow[j] >= 5 || nrow[j] == 0 ? 0
              : (nrow[j] >= 3 ? 1 : (nrow[j] == 2 ? 2 : 3));
    }
    int off[SLOTS];   // lane s < 2K: sweep_range[row][s]
    int hrow[SLOTS];  // REPLAY 4: the row of A^T (a piece's own row) whose h_{t-1} the group's dots read, or -1
#pragma unroll
    for (int j = 0; j < SLOTS; ++j) {
      const int i = g >> lf[j];
      const int32_t rj = i < nrow[j] ? row_at(base + 8u * j + (uint32_t)i) : -1;
      off[j] = rj >= 0 && s < 2 * K ? a.sweep_range[(int64_t)rj * (2 * K) + s] : 0;
      if constexpr (REPLAY == 4) hrow[j] = rj < 0 ? -1 : (rj < a.nrows ? rj : a.piece_row[rj - a.nrows]);
      if constexpr (REPLAY != 1) {
        // the epilogue's row (first group of a spread row only) and word s of its constants, for every chunk
        const bool first = (g & ((1 << lf[j]) - 1)) == 0;
        const int e = (wv * SLOTS + j) * 64 + lane;
        ep_row[e] = first ? rj : -1;
        if constexpr (REPLAY != 3 && REPLAY != 4)
          ep_par[e] = first && rj >= 0 && rj < a.nrows ? reinterpret_cast<const int *>(a.params + rj)[s] : 0;
      }
    }
    for (int c = 0; c < chunks; ++c) {
      const int64_t col = (int64_t)c * (8 * V) + (int64_t)s * V;
      const bool in_batch = col < a.batch;
      // lanes past the batch gather their chunk's first columns (no sum reads them), or zeros where a record's
      // dot sums the group's columns (an offset past any buffer below 2^31 bytes)
      const uint32_t voff = REPLAY == 4 ? (in_batch ? (uint32_t)col * (uint32_t)sizeof(S) : 0x80000000u)
                                        : (uint32_t)(in_batch ? col : (int64_t)c * (8 * V)) * (uint32_t)sizeof(S);
      float hv[REPLAY == 4 ? SLOTS : 1][V];   // REPLAY 4: the group's row of h_{t-1}, this lane's columns
      if constexpr (REPLAY == 4) {
#pragma unroll
        for (int j = 0; j < SLOTS; ++j) {
          if (hrow[j] >= 0 && in_batch) {
            Lanes<float, V>::load(a.hdot + (int64_t)hrow[j] * a.ldh + col, hv[j]);
          } else {
#pragma unroll
            for (int i = 0; i < V; ++i) hv[j][i] = 0.0f;
          }
        }
      }
      float acc[SLOTS][V];
#pragma unroll
      for (int j = 0; j < SLOTS; ++j)
#pragma unroll
        for (int i = 0; i < V; ++i) acc[j][i] = 0.0f;
      // slot 0's first records of the next band, loaded with the band's last slot (see below)
      int2 pre_next[3];
      static_for<K>([&](auto B) {
        constexpr int b = decltype(B)::value;
        if constexpr (PAIRED) {
          // Two slots' rows per pass: the group walks row A's band-b non-zeros, then row B's, so a pass runs to
          // the longest pair of the wave's 8 instead of each slot to its longest row; every gathered row feeds the
          // sums of the row it belongs to (the other row's weight is zero).
#pragma unroll
          for (int j = 0; j < SLOTS; j += 2) {
            const int bA = group_bcast<8, 2 * b>(off[j]), eA = group_bcast<8, 2 * b + 1>(off[j]);
            const int bB = group_bcast<8, 2 * b>(off[j + 1]), eB = group_bcast<8, 2 * b + 1>(off[j + 1]);
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
                      if constexpr (PAIRED == 2) {
                        // only the row that owns the gathered record changes: a zero weight times an inf or NaN
                        // source would otherwise reach the partner row, which never reads that source
#pragma unroll
                        for (int i = 0; i < V; ++i) {
                          const float x = Lanes<S, V>::at(xr[u], i);
                          const float ta = fmaf(wt, x, acc[j][i]), tb = fmaf(wt, x, acc[j + 1][i]);
                          acc[j][i] = in_a ? ta : acc[j][i];
                          acc[j + 1][i] = in_a ? acc[j + 1][i] : tb;
                        }
                      } else {
                        // the other row's weight is zero: exact for the finite states of a bounded clamp
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
                }
              });
              rec = nxt;
            }
          }
        } else {
#pragma unroll
        for (int j = 0; j < SLOTS; ++j) {
          int beg = group_bcast<8, 2 * b>(off[j]), end = group_bcast<8, 2 * b + 1>(off[j]);
          if (lf[j]) {   // this group's share of the row's band
            const int n = end - beg, p = g & ((1 << lf[j]) - 1), b0 = beg;
            beg = b0 + ((n * p) >> lf[j]);
            end = b0 + ((n * (p + 1)) >> lf[j]);
          }
          const int rounds = wave_max_of_groups(end - beg);
          // lane s brings record q0 + s of its row's band (clamped into the row), and round q reaches the group's
          // lanes by a broadcast of lane q (the first blocks of a slot load together, below)
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
          // one block of 8 rounds: the gathers and sums of records rec (lane s: record q0 + s of its group's row)
          auto run_block = [&](const int2 rec, int q0) {
            float dl[REPLAY == 4 ? 8 : 1];   // REPLAY 4: this lane's share of each round's dot
#pragma unroll
            for (int u = 0; u < (REPLAY == 4 ? 8 : 1); ++u) dl[u] = 0.0f;
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
                    if constexpr (REPLAY == 4) {
                      float d = 0.0f;
#pragma unroll
                      for (int i = 0; i < V; ++i) d = fmaf(Lanes<S, V>::at(xr[u], i), hv[j][i], d);
                      dl[h0 + u] = d;
                    }
                  }
                }
              }
            });
            if constexpr (REPLAY == 4) {
              // lane s ends with the group's dot of round s: the record it loaded for this block
              const float dot = group_reduce_scatter8(dl, s);
              const int q = beg + q0 + s;
              if (q < end) __builtin_nontemporal_store(dot, a.dots + (int64_t)c * a.ndots + q);
            }
          };
          // The first blocks' records load together (PRE blocks, 6 VGPRs): vector memory counters retire in order,
          // so a record load issued during a block's gathers holds up that block's sums, and one shared wait per
          // slot and band replaces one per block.  Longer bands go on block by block, the next one's load in flight.
          // (The training backward's pass, whose dots hold more registers, keeps the next block's load in flight
          // from the start instead: 3 blocks spill there.)
          constexpr int PRE = REPLAY == 4 ? 0 : 3;
          int2 pre[PRE > 0 ? PRE : 1];
          if (PRE > 0 && b > 0 && j == 0) {
            // loaded with the previous band's last slot, so the wait for them is not the first thing after the
            // workgroup's barrier
#pragma unroll
            for (int kb = 0; kb < (PRE > 0 ? PRE : 1); ++kb) pre[kb] = pre_next[kb];
          } else {
            static_for<PRE>([&](auto KB) {
              constexpr int kb = decltype(KB)::value;
              pre[kb] = kb * 8 < rounds ? block(kb * 8) : make_int2(0, 0);
            });
          }
          if constexpr (PRE == 3 && b + 1 < K) {
            if (j == SLOTS - 1) {   // slot 0's first records of the next band, issued with this slot's own
              int nb = group_bcast<8, 2 * (b + 1)>(off[0]), ne = group_bcast<8, 2 * (b + 1) + 1>(off[0]);
              if (lf[0]) {
                const int n = ne - nb, p = g & ((1 << lf[0]) - 1), b0 = nb;
                nb = b0 + ((n * p) >> lf[0]);
                ne = b0 + ((n * (p + 1)) >> lf[0]);
              }
              const int r1 = wave_max_of_groups(ne - nb);
              static_for<3>([&](auto KB) {
                constexpr int kb = decltype(KB)::value;
                if (kb * 8 < r1) {
                  const int q = nb + kb * 8 + s;
                  const int2 rc = a.colval[max(min(q, ne - 1), 0)];
                  pre_next[kb] = q < ne ? rc : make_int2((int)past_row, 0);
                } else {
                  pre_next[kb] = make_int2(0, 0);
                }
              });
            }
          }
          static_for<PRE>([&](auto KB) {
            constexpr int kb = decltype(KB)::value;
            if (kb * 8 < rounds) run_block(pre[kb], kb * 8);
          });
          if (rounds > PRE * 8) {
            int2 rec = block(PRE * 8);
            for (int q0 = PRE * 8; q0 < rounds; q0 += 8) {
              const int2 nxt = block(q0 + 8);
              run_block(rec, q0);
              rec = nxt;
            }
          }
          }
        }
        }
        // the workgroup's waves start the next band together; after the last band each wave goes on to its epilogue
        // and the next chunk's first band at once, so its row reads and stores overlap the slower waves' gathers
        // (state steps 4.700 -> 4.630 ms per forward at B = 1120), and they meet again after that band
        if (b + 1 < K || a.sweep_last_sync > 0) __syncthreads();
      });
      if constexpr (REPLAY != 1) {
#pragma unroll
        for (int j = 0; j < SLOTS; ++j) {
          if (lf[j]) {   // the shares of a spread row meet in each of its groups
#pragma unroll
            for (int i = 0; i < V; ++i) acc[j][i] = groups_sum(acc[j][i], lf[j]);
          }
        }
        // Slots in batches: the carried state and drive of a batch's rows load together, then the batch finishes.
        // Batches of 3, or of 2 when 6 slots' sums share the registers with 32-byte drive vectors (float32 drive
        // of a half state), which would otherwise spill.
        constexpr int EB = (SLOTS == 6 && V * sizeof(U) > 16) ? 2 : (SLOTS % 3 == 0 ? 3 : 1);
        // A batch's new states are stored after the next batch's loads are issued: vector memory counters retire
        // in order, so the next batch's epilogue then waits for its own loads and not for these stores.  (Not
        // with 6 slots of a half state and half drive, whose batches of 3 rows would spill the held states.)
        constexpr bool DEFER = (REPLAY == 0 || REPLAY == 2) && !(sizeof(S) == 2 && sizeof(U) == 2 && SLOTS == 6);
        constexpr int NP = DEFER ? EB : 1;
        typename Lanes<S, V>::vec pend[NP];
        int prow[NP];
#pragma unroll
        for (int u = 0; u < NP; ++u) prow[u] = -1;
        auto flush = [&]() {
#pragma unroll
          for (int u = 0; u < NP; ++u) {
            if (prow[u] >= 0) Lanes<S, V>::store_raw(a.xout + (int64_t)prow[u] * a.ldo + col, pend[u], a.nt_store != 0);
            prow[u] = -1;
          }
        };
        static_for<SLOTS / EB>([&](auto H) {
          constexpr int j0 = decltype(H)::value * EB;
          int rs[EB];
          RowInputs<S, U, V> in[EB];
          static_for<EB>([&](auto J) {
            constexpr int u = decltype(J)::value;
            const int e = (wv * SLOTS + j0 + u) * 64 + lane;
            rs[u] = in_batch ? ep_row[e] : -1;
            if constexpr (REPLAY != 3 && REPLAY != 4) {
              in[u].p = row_param_from_word(ep_par[e]);   // every lane takes part in the group broadcasts
              load_row_drive(a, col, rs[u] >= 0 && rs[u] < a.nrows, in[u]);
            }
          });
          if constexpr (DEFER) flush();
          static_for<EB>([&](auto J) {
            constexpr int u = decltype(J)::value;
            if (rs[u] >= a.nrows) {   // a piece of a split row: its raw sums
              if constexpr (REPLAY != 2) {
                float *dst = a.pieces + (int64_t)(rs[u] - a.nrows) * a.ldp + col;
                Lanes<float, V>::store(dst, acc[j0 + u]);
              }
            } else if (rs[u] >= 0) {
              const uint32_t rj = (uint32_t)rs[u];
              if constexpr (REPLAY == 3 || REPLAY == 4) {   // the product alone: y[row] (+)= the row's sums, float32
                S *dst = a.xout + (int64_t)rj * a.ldo + col;
                if (a.accumulate) {
                  float o[V];
                  Lanes<float, V>::load(dst, o);
#pragma unroll
                  for (int i = 0; i < V; ++i) acc[j0 + u][i] += o[i];
                }
                Lanes<S, V>::store(dst, acc[j0 + u]);
              } else {
                if constexpr (REPLAY == 2) ReplayBits<S, V>::seed(acc[j0 + u], bits);
                if constexpr (DEFER) {
                  float out[V];
                  finish_value<S, U, V, TORCH_LERP>(a, col, acc[j0 + u], in[u], out);
                  pend[u % NP] = Lanes<S, V>::pack(out);
                  prow[u % NP] = (int)rj;
                } else {
                  finish_row<S, U, V, TORCH_LERP>(a, rj, col, acc[j0 + u], in[u]);
                }
              }
            }
          });
        });
        if constexpr (DEFER) flush();
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

// The rows a swept step split into pieces (k_state_step_swept stored each piece's raw sums): per split row, the
// pieces' sums added in piece order, then the row's epilogue as the swept kernel runs it (REPLAY == 3 and 4: the
// sums stored, or added with a.accumulate).  One thread per V columns of a row, blockIdx.y over the split rows.
template <typename S, typename U, int V, bool TORCH_LERP, int REPLAY>
__global__ __launch_bounds__(256) void k_sweep_finish(const StepArgs<S, U> a, const int32_t *__restrict__ split,
                                                     const int32_t *__restrict__ split_ptr, int32_t nsplit) {
  const int64_t col = (blockIdx.x * (int64_t)blockDim.x + threadIdx.x) * V;
  if (col >= a.batch) return;
  for (int32_t h = blockIdx.y; h < nsplit; h += gridDim.y) {
    float acc[V];
#pragma unroll
    for (int i = 0; i < V; ++i) acc[i] = 0.0f;
    const int32_t q1 = split_ptr[h + 1];
    for (int32_t q = split_ptr[h]; q < q1; ++q) {
      float v[V];
      Lanes<float, V>::load(a.pieces + (int64_t)q * a.ldp + col, v);
#pragma unroll
      for (int i = 0; i < V; ++i) acc[i] += v[i];
    }
    const uint32_t row = (uint32_t)split[h];
    if constexpr (REPLAY == 3 || REPLAY == 4) {
      S *dst = a.xout + (int64_t)row * a.ldo + col;
      if (a.accumulate) {
        float o[V];
        Lanes<float, V>::load(dst, o);
#pragma unroll
        for (int i = 0; i < V; ++i) acc[i] += o[i];
      }
      Lanes<S, V>::store(dst, acc);
    } else {
      RowInputs<S, U, V> in;
      load_row_inputs(a, row, col, true, in);
      finish_row<S, U, V, TORCH_LERP>(a, row, col, acc, in);
    }
  }
}

template <typename S, typename U, int K, int SLOTS, int REPLAY, int PAIRED = 0, bool PIPE = false>
void launch_swept_shape(const StepArgs<S, U> &a, unsigned grid, hipStream_t st) {
  constexpr int V = 16 / (int)sizeof(S);
  static std::atomic<bool> fits{false};
  if (!fits.load(std::memory_order_relaxed)) {   // the kernel's registers allow one 16-wave workgroup on a CU
    int nb = 0;
    FLY_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(
        &nb,
        reinterpret_cast<const void *>(&k_state_step_swept<S, U, V, K, SLOTS, sizeof(S) == 4, REPLAY, PAIRED, PIPE>),
        1024, 0));
    FLY_REQUIRE(nb >= 1, "the swept state step does not fit a CU");
    fits.store(true, std::memory_order_relaxed);
  }
  hipLaunchKernelGGL((k_state_step_swept<S, U, V, K, SLOTS, sizeof(S) == 4, REPLAY, PAIRED, PIPE>), dim3(grid),
                     dim3(1024), 0, st, a);
}

// Bytes of the pieces buffer a swept step of `batch` columns over these tables needs (0 without split rows).
inline size_t sweep_pieces_bytes(const SweepTables *t, int64_t batch) {
  return t && t->pieces ? (size_t)t->pieces * (size_t)round_up(batch, 64) * sizeof(float) : 0;
}

// One swept step over the tables of its structure: one workgroup per CU (or the tables' grid), the rows split evenly
// between the waves (one pass of up to 24 or 48 rows per wave; a larger step takes several passes), then the split
// rows' pieces added and finished.  a.pieces: sweep_pieces_bytes(t, batch) bytes, 16-byte aligned (unused without
// split rows).
template <typename S, typename U, int REPLAY>
void launch_swept(StepArgs<S, U> a, const SweepTables &t, hipStream_t st) {
  FLY_REQUIRE(t.nrows == a.nrows, "sweep tables of another structure");
  FLY_REQUIRE(!t.pieces || REPLAY == 1 || REPLAY == 2 || (a.pieces && aligned(a.pieces, 32)),
              "a swept step with split rows needs its pieces buffer");
  const unsigned grid = (unsigned)t.grid;
  a.sweep_range = t.range.p;
  a.sweep_order = t.order.p;
  a.sweep_npos = (int32_t)t.npos;
  a.sweep_vrows = (int32_t)(t.nrows + t.pieces);
  a.rows_per_wave = t.rows_per_wave;
  a.ldp = round_up(a.batch, 64);
  const bool few = a.rows_per_wave <= 24 || a.sweep_slots == 3;
  if constexpr (REPLAY == 4) {
    // the transposed backward keeps each slot's row of h_{t-1} beside its sums
    static_assert(sizeof(S) == 4, "the transposed backward is float32");
    if (t.bands == 3) {
      if (few) launch_swept_shape<S, U, 3, 3, 4>(a, grid, st);
      else launch_swept_shape<S, U, 3, 6, 4>(a, grid, st);
    } else {
      if (few) launch_swept_shape<S, U, 4, 3, 4>(a, grid, st);
      else launch_swept_shape<S, U, 4, 6, 4>(a, grid, st);
    }
  } else {
  switch (t.bands) {
    case 3:
      if (few) launch_swept_shape<S, U, 3, 3, REPLAY>(a, grid, st);
      else launch_swept_shape<S, U, 3, 6, REPLAY>(a, grid, st);
      break;
    case 4:
      // passes of 3 slots keep the next four rounds' gathers in flight during the sums (step 5 at B = 1120:
      // 1.006 -> 0.959 ms); at 6 slots the second set of gathers costs spills and gains nothing
      if (few && a.sweep_pipe >= 0) launch_swept_shape<S, U, 4, 3, REPLAY, 0, true>(a, grid, st);
      else if (few) launch_swept_shape<S, U, 4, 3, REPLAY>(a, grid, st);
      else if (a.sweep_pipe > 0) launch_swept_shape<S, U, 4, 6, REPLAY, 0, true>(a, grid, st);
      // two rows per pass only when the tuning asks: with the epilogue's batched loads one row per pass measured
      // faster for float32 states too (126,100 against 124,500 evals/s, float32 light cone at B = 1120), and half
      // states lose 5% (16 FMAs per gathered line of 8 halves cost more than the rounds they save)
      else if (a.sweep_paired > 0) {
        if (a.sweep_exact) launch_swept_shape<S, U, 4, 6, REPLAY, 2>(a, grid, st);
        else launch_swept_shape<S, U, 4, 6, REPLAY, 1>(a, grid, st);
      } else {
        launch_swept_shape<S, U, 4, 6, REPLAY>(a, grid, st);
      }
      break;
    default:
      FLY_REQUIRE(false, "swept steps take 3 or 4 bands");
  }
  }
  if (t.pieces && (REPLAY == 0 || REPLAY == 3 || REPLAY == 4)) {
    constexpr int V = 16 / (int)sizeof(S);
    const dim3 fgrid(blocks_for((a.batch + V - 1) / V, 256), (unsigned)std::min<int64_t>(t.split_rows, 65535));
    hipLaunchKernelGGL((k_sweep_finish<S, U, V, sizeof(S) == 4, REPLAY>), fgrid, dim3(256), 0, st, a, t.split.p,
                       t.split_ptr.p, (int32_t)t.split_rows);
  }
}

// ---- lead row slots --------------------------------------------------------------------------------------

namespace {
// flag[s] = 1 where a slot of 8 consecutive rows holds a row of more than len non-zeros
__global__ __launch_bounds__(256) void k_lead_flags(const int32_t *__restrict__ rowptr, int64_t nrows, int64_t slots,
                                                    int32_t len, uint8_t *__restrict__ flag) {
  const int64_t sl = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (sl >= slots) return;
  int32_t longest = 0;
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    const int64_t row = sl * 8 + r;
    if (row < nrows) longest = max(longest, rowptr[row + 1] - rowptr[row]);
  }
  flag[sl] = longest > len ? 1 : 0;
}
}  // namespace

struct LeadSlots {
  DevArray<int32_t> lead;    // the lead slots, rising
  DevArray<uint8_t> flag;    // (slots of 8 rows) 1 for a lead slot
  int32_t n = 0;
};

// The lead slots of a step matrix (rowptr, nrows + 1) whose rows run as slots of 8 rows: those holding a row of more
// than max(64, 8 x the mean) non-zeros (on the real connectome's in-degrees, step 2's rows average 7.6 non-zeros
// and reach 1,008).  Synchronises the stream: the count sizes the launch.  None (n = 0) for an empty matrix.
inline LeadSlots build_lead_slots(const int32_t *rowptr, int64_t nrows, int64_t nnz, hipStream_t st) {
  LeadSlots out;
  if (!rowptr || nrows <= 0 || nnz <= 0) return out;
  const int64_t slots = (nrows + 7) / 8;
  const int32_t len = (int32_t)std::min<int64_t>(INT32_MAX, std::max<int64_t>(64, 8 * nnz / nrows));
  DevArray<uint8_t> flag(slots);
  hipLaunchKernelGGL(k_lead_flags, dim3(blocks_for(slots, 256)), dim3(256), 0, st, rowptr, nrows, slots, len, flag.p);
  FLY_HIP(hipGetLastError());
  std::vector<uint8_t> hf(slots);
  FLY_HIP(hipMemcpyAsync(hf.data(), flag.p, (size_t)slots, hipMemcpyDeviceToHost, st));
  FLY_HIP(hipStreamSynchronize(st));
  std::vector<int32_t> list;
  for (int64_t i = 0; i < slots; ++i)
    if (hf[i]) list.push_back((int32_t)i);
  if (list.empty()) return out;
  out.lead.alloc(list.size());
  FLY_HIP(hipMemcpyAsync(out.lead.p, list.data(), sizeof(int32_t) * list.size(), hipMemcpyHostToDevice, st));
  FLY_HIP(hipStreamSynchronize(st));   // the host list is a temporary
  out.flag = std::move(flag);
  out.n = (int32_t)list.size();
  return out;
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
  a.nt_load = tune.nt_load;
  a.slots = sh.rows_mode ? (a.nrows + sh.groups - 1) / sh.groups : a.nrows;
  return sh;
}

}  // namespace fly
