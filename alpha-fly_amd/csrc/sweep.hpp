// Banded-sweep tables of one CSR structure, built once per structure on the device, and the rule for when a matrix
// sweeps.  Shared by the evaluator library and the bench's measurement library.
//
// A swept step's waves take the matrix's rows in an order of positions (`order`); each position holds a row, or a
// piece of a row the tables split because it is far longer than the mean (a hub of a heavy-tailed in-degree).  A
// piece takes an equal share of each of its row's bands, so to the sweep it is one more row of ordinary length; it
// stores its raw sums, and the step adds a split row's pieces in piece order before that row's epilogue.  Per row
// of the order (rows, then pieces) `range` holds, for each band b of source rows, where that row's records of band b
// begin and end: band b holds the source rows [b * ncols / K, (b + 1) * ncols / K).
#pragma once

#include <algorithm>
#include <atomic>
#include <cstring>
#include <functional>
#include <memory>
#include <mutex>
#include <queue>
#include <vector>

#include "common.hpp"
#include "device.hpp"

namespace fly {

constexpr int kSweepBands = 4;   // source bands of a swept step: 3 and 4 measured best (5: +3%, 6: +6% per step)

// Whether a step runs as a banded sweep by size: its sources overflow one XCD's 4 MB L2 at one 128-byte line per row
// and chunk (more than 32,768 rows of X_{t-1}), it has rows enough to give each of the GPU's waves several, and its
// rows are long enough for every band to hold several non-zeros.
inline bool sweep_eligible(int64_t prev_rows, int64_t rows, int64_t nnz) {
  return prev_rows > 32768 && rows >= 65536 && nnz >= 32 * rows;
}

// How a structure's tables are built (captured from the tuning when a plan or fly_sweep is created).
struct SweepConfig {
  int32_t bands = kSweepBands;   // 3 or 4
  int32_t paired = 0;            // the order is searched for waves that walk two slots per pass (float32 states)
  int32_t grid = 0;              // workgroups of the swept launch; 0: one per CU of the current device
  int32_t force = 0;             // sweep any matrix with rows and non-zeros, whatever its size
  int32_t piece = 0;             // split rows longer than this into pieces of at most this many non-zeros; 0: 3 x the
                                 // mean + 10
  int32_t search = 1;            // 0: the initial order, unsorted and unsearched
  int32_t deal = 0;              // the initial order dealt out by work: 0 where index order is unbalanced, 1 always,
                                 // -1 never
  bool operator==(const SweepConfig &o) const { return std::memcmp(this, &o, sizeof(*this)) == 0; }
};

struct SweepTables {
  int32_t bands = kSweepBands, paired = 0, grid = 0, rows_per_wave = 0;
  int32_t dealt = 0;                // the initial order was dealt out by work (the index order was unbalanced)
  int64_t nrows = 0, ncols = 0, nnz = 0;
  int64_t npos = 0;                 // positions of the order: the rows not split, plus the pieces
  int64_t pieces = 0, split_rows = 0;
  DevArray<int32_t> range;          // (nrows + pieces, 2 * bands)
  DevArray<int32_t> order;          // (npos): a row (< nrows) or nrows + a piece
  DevArray<int32_t> split;          // (split_rows): the rows split into pieces
  DevArray<int32_t> split_ptr;      // (split_rows + 1): the pieces of split[h] are split_ptr[h] .. split_ptr[h + 1] - 1
  DevArray<int32_t> piece_row;      // (pieces): the row each piece belongs to
};

// The GPU's CU count (the swept kernel runs one workgroup per CU), per device, cached; safe to call from several
// threads (a first call that races computes the same value).
inline int cu_count() {
  static std::atomic<int> cached[64];
  const int dev = current_device();
  if (dev >= 0 && dev < 64) {
    const int n = cached[dev].load(std::memory_order_relaxed);
    if (n > 0) return n;
  }
  int cus = 0;
  FLY_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  FLY_REQUIRE(cus > 0, "no compute units");
  if (dev >= 0 && dev < 64) cached[dev].store(cus, std::memory_order_relaxed);
  return cus;
}

namespace {


// Per row of A_t, where each of K bands of source rows begins among its non-zeros: band b holds the columns
// [b * prev_rows / K, (b + 1) * prev_rows / K).  off (nr, K + 1): the row's start plus the count of its columns in
// the bands before b; off[i][K] is the row's end.  A row's columns rise (CSR order of W[post, pre]), so each range
// holds exactly its band; in any other order the ranges still split the row's non-zeros between the bands.
__device__ __forceinline__ int32_t record_col(const int2 &r) { return r.x; }
__device__ __forceinline__ int32_t record_col(int32_t c) { return c; }

template <typename C>   // C: {column, weight} records (int2) or plain columns (int32_t)
__global__ __launch_bounds__(256) void k_band_off(const int32_t *__restrict__ rowptr, const C *__restrict__ colval,
                                                  int64_t nr, int64_t prev_rows, int32_t K, int32_t *__restrict__ off) {
  // 16 lanes per row, lane s counting the records s, s + 16, ..., their counts added through xor shuffles (a hub
  // row's thousands of records do not fall to one lane)
  const int s = threadIdx.x & 15;
  const int64_t i = blockIdx.x * 16 + (threadIdx.x >> 4);
  const bool has = i < nr;
  const int32_t beg = has ? rowptr[i] : 0, end = has ? rowptr[i + 1] : 0;
  int32_t cnt[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int32_t q = beg + s; q < end; q += 16) {
    const int64_t b = (int64_t)record_col(colval[q]) * K / prev_rows;
#pragma unroll
    for (int k = 0; k < 8; ++k) cnt[k] += (b == k) ? 1 : 0;
  }
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    cnt[k] += __shfl_xor(cnt[k], 8);
    cnt[k] += __shfl_xor(cnt[k], 4);
    cnt[k] += __shfl_xor(cnt[k], 2);
    cnt[k] += __shfl_xor(cnt[k], 1);
  }
  if (!has || s != 0) return;
  int32_t o = beg;
  for (int k = 0; k < K; ++k) {
    off[i * (K + 1) + k] = o;
    o += cnt[k];
  }
  off[i * (K + 1) + K] = end;
}

// The order in which the swept kernel's waves take a step's rows: each wave's own `per` consecutive positions of the
// initial order `in`, longest first (ties in initial order), into `out`, so the 8 rows of a slot are of like length
// and its rounds, which run to the longest of them, waste fewer gathers, while every wave keeps the same rows and
// share of the work.  One thread per wave's segment ranks each of its rows by counting the rows that go before it.
// A row's length is the sum of its band ranges (range: (rows, 2K) begin/end pairs).
__global__ void k_sweep_order(const int32_t *__restrict__ range, int K, const int32_t *__restrict__ in, int64_t npos,
                              int64_t per, int32_t *__restrict__ out) {
  const int64_t seg = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  const int64_t b = seg * per;
  if (b >= npos) return;
  const int64_t e = min(b + per, npos);
  auto len = [&](int64_t p) {
    const int32_t *r = range + (int64_t)in[p] * (2 * K);
    int32_t n = 0;
    for (int q = 0; q < K; ++q) n += r[2 * q + 1] - r[2 * q];
    return n;
  };
  for (int64_t i = b; i < e; ++i) {
    const int32_t li = len(i);
    int64_t rank = 0;
    for (int64_t j = b; j < e; ++j) {
      const int32_t lj = len(j);
      rank += (lj > li || (lj == li && j < i)) ? 1 : 0;
    }
    out[b + rank] = in[i];
  }
}

// k_sweep_order with one 64-lane workgroup per wave's segment and the segment's lengths in LDS (per ints of dynamic
// LDS): the same ranks, each lane ranking positions i, i + 64, ... against the lengths in LDS instead of summing
// every other position's band ranges again from memory.
__global__ __launch_bounds__(64) void k_sweep_order_lds(const int32_t *__restrict__ range, int K,
                                                        const int32_t *__restrict__ in, int64_t npos, int64_t per,
                                                        int32_t *__restrict__ out) {
  extern __shared__ int32_t seg_len[];
  const int64_t b = (int64_t)blockIdx.x * per;
  if (b >= npos) return;
  const int m = (int)min(per, npos - b);
  for (int k = threadIdx.x; k < m; k += 64) {
    const int32_t *r = range + (int64_t)in[b + k] * (2 * K);
    int32_t n = 0;
    for (int q = 0; q < K; ++q) n += r[2 * q + 1] - r[2 * q];
    seg_len[k] = n;
  }
  __syncthreads();
  for (int i = threadIdx.x; i < m; i += 64) {
    const int32_t li = seg_len[i];
    int rank = 0;
    for (int j = 0; j < m; ++j) {
      const int32_t lj = seg_len[j];
      rank += (lj > li || (lj == li && j < i)) ? 1 : 0;
    }
    out[b + rank] = in[b + i];
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
__global__ __launch_bounds__(64) void k_sweep_order_search(const int32_t *__restrict__ range, int K, int64_t nr,
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
      cnt[q][k] = (uint16_t)min(range[(int64_t)r * (2 * K) + 2 * q + 1] - range[(int64_t)r * (2 * K) + 2 * q], 65535);
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
__global__ __launch_bounds__(kBalanceThreads) void k_sweep_order_balance(const int32_t *__restrict__ range, int K,
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
      cnt[q][p] = (uint16_t)min(range[(int64_t)r * (2 * K) + 2 * q + 1] - range[(int64_t)r * (2 * K) + 2 * q], 65535);
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


// A piece of a split row: the row, the piece's index among the row's pieces and their count.
struct PieceDesc {
  int32_t row, index, count, pad;
};

// range (rows + pieces, 2K) from the per-row band starts off (rows, K + 1): a row's band b is [off[b], off[b + 1]); a
// piece i of m of row h takes [off[b] + n_b i / m, off[b] + n_b (i + 1) / m) of each band (n_b: the row's band count).
__global__ void k_sweep_ranges(const int32_t *__restrict__ off, int K, int64_t nrows,
                               const PieceDesc *__restrict__ pieces, int64_t npieces, int32_t *__restrict__ range) {
  const int64_t v = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (v >= nrows + npieces) return;
  int32_t *out = range + v * (2 * K);
  if (v < nrows) {
    for (int b = 0; b < K; ++b) {
      out[2 * b] = off[v * (K + 1) + b];
      out[2 * b + 1] = off[v * (K + 1) + b + 1];
    }
    return;
  }
  const PieceDesc d = pieces[v - nrows];
  for (int b = 0; b < K; ++b) {
    const int64_t o = off[(int64_t)d.row * (K + 1) + b], n = off[(int64_t)d.row * (K + 1) + b + 1] - o;
    out[2 * b] = (int32_t)(o + n * d.index / d.count);
    out[2 * b + 1] = (int32_t)(o + n * (d.index + 1) / d.count);
  }
}

}  // namespace

// The tables of one CSR structure (rowptr nrows + 1, records or columns nnz, columns below ncols), or null when it
// does not sweep (by size, unless cfg.force).  Synchronises the stream (it reads the row lengths back).
//   1. Rows longer than the limit are split into pieces (host), each taking a share of every band.
//   2. Band starts per row (k_band_off), then the range table of rows and pieces (k_sweep_ranges).
//   3. The initial order: the unsplit rows in index order, with the pieces at evenly spaced positions among them.
//   4. Each wave's rows longest first (k_sweep_order), then rearranged between the wave's slots
//      (k_sweep_order_search) and between the 16 waves of each workgroup (k_sweep_order_balance).
template <typename C>
std::shared_ptr<SweepTables> build_sweep(const int32_t *rowptr, const C *cols, int64_t nrows, int64_t nnz,
                                         int64_t ncols, const SweepConfig &cfg, hipStream_t st) {
  FLY_REQUIRE(cfg.bands == 3 || cfg.bands == 4, "swept steps take 3 or 4 bands");
  if (nrows <= 0 || nnz <= 0 || ncols <= 0) return nullptr;
  if (!cfg.force && !sweep_eligible(ncols, nrows, nnz)) return nullptr;
  FLY_REQUIRE(nrows < (int64_t)1 << 24 && ncols < (int64_t)1 << 24 && nnz < (int64_t)INT32_MAX,
              "swept structures hold below 2^24 rows and columns");
  const int K = cfg.bands;
  std::vector<int32_t> rp((size_t)nrows + 1);
  FLY_HIP(hipMemcpyAsync(rp.data(), rowptr, sizeof(int32_t) * rp.size(), hipMemcpyDeviceToHost, st));
  FLY_HIP(hipStreamSynchronize(st));
  FLY_REQUIRE(rp[0] == 0 && rp[nrows] == nnz, "the row pointer does not span the non-zeros");
  // 1. split rows
  //    Rows over 3 x the mean + 10 non-zeros run to several times their slot's other rows (measured on the real
  //    connectome's in-degrees at B = 1120: limits of 120, 150, 180, 200 (3 x the mean + 10), 230 and 260 gave state
  //    steps of 5.77, 5.58, 5.55, 5.49, 5.62 and 6.32 ms per forward).
  const double mean = (double)nnz / (double)nrows;
  const int64_t limit = cfg.piece > 0 ? cfg.piece : std::max<int64_t>(8, (int64_t)(3.0 * mean + 10.0));
  const int64_t piece = limit;
  std::vector<PieceDesc> pieces;
  std::vector<int32_t> split, split_ptr{0};
  std::vector<uint8_t> is_split((size_t)nrows, 0);
  for (int64_t r = 0; r < nrows; ++r) {
    const int64_t len = rp[r + 1] - rp[r];
    if (len <= limit) continue;
    const int32_t m = (int32_t)((len + piece - 1) / piece);
    for (int32_t i = 0; i < m; ++i) pieces.push_back({(int32_t)r, i, m, 0});
    split.push_back((int32_t)r);
    split_ptr.push_back((int32_t)pieces.size());
    is_split[r] = 1;
  }
  auto t = std::make_shared<SweepTables>();
  t->bands = K;
  t->grid = cfg.grid > 0 ? cfg.grid : cu_count();
  t->nrows = nrows;
  t->ncols = ncols;
  t->nnz = nnz;
  t->pieces = (int64_t)pieces.size();
  t->split_rows = (int64_t)split.size();
  t->npos = nrows - t->split_rows + t->pieces;
  FLY_REQUIRE(nrows + t->pieces < (int64_t)1 << 24, "too many pieces");
  // 2. ranges
  std::vector<int32_t> prow;   // each piece's row (copied until the synchronisation below)
  {
    DevArray<int32_t> off((size_t)nrows * (K + 1));
    hipLaunchKernelGGL(k_band_off<C>, dim3(blocks_for(nrows, 16)), dim3(256), 0, st, rowptr, cols, nrows, ncols, K,
                       off.p);
    DevArray<PieceDesc> pd(pieces.size());
    if (!pieces.empty())
      FLY_HIP(hipMemcpyAsync(pd.p, pieces.data(), sizeof(PieceDesc) * pieces.size(), hipMemcpyHostToDevice, st));
    t->range.alloc((size_t)(nrows + t->pieces) * 2 * K);
    hipLaunchKernelGGL(k_sweep_ranges, dim3(blocks_for(nrows + t->pieces, 256)), dim3(256), 0, st, off.p, K, nrows,
                       pd.p, t->pieces, t->range.p);
    check_launch("sweep ranges");
    if (!split.empty()) {
      t->split.alloc(split.size());
      t->split_ptr.alloc(split_ptr.size());
      FLY_HIP(hipMemcpyAsync(t->split.p, split.data(), sizeof(int32_t) * split.size(), hipMemcpyHostToDevice, st));
      FLY_HIP(hipMemcpyAsync(t->split_ptr.p, split_ptr.data(), sizeof(int32_t) * split_ptr.size(),
                             hipMemcpyHostToDevice, st));
      prow.resize(pieces.size());
      for (size_t q = 0; q < pieces.size(); ++q) prow[q] = pieces[q].row;
      t->piece_row.alloc(prow.size());
      FLY_HIP(hipMemcpyAsync(t->piece_row.p, prow.data(), sizeof(int32_t) * prow.size(), hipMemcpyHostToDevice, st));
    }
    FLY_HIP(hipStreamSynchronize(st));   // the host vectors and temporaries end here
  }
  // 3. initial order: piece j at position floor((2 j + 1) npos / (2 pieces)), the unsplit rows in index order between
  std::vector<int32_t> ord((size_t)t->npos);
  {
    int64_t j = 0, r = 0;
    for (int64_t p = 0; p < t->npos; ++p) {
      if (j < t->pieces && p == (2 * j + 1) * t->npos / (2 * t->pieces)) {
        ord[p] = (int32_t)(nrows + j++);
      } else {
        while (is_split[r]) ++r;
        ord[p] = (int32_t)r++;
      }
    }
  }
  const int64_t waves = 16 * (int64_t)t->grid;
  const int64_t per = (t->npos + waves - 1) / waves;   // the launch's rows_per_wave
  const int64_t segs = (t->npos + per - 1) / per;
  //    A workgroup waits for its slowest wave and the step for its slowest workgroup.  Where rows of like length sit
  //    together in index order (a real connectome's neurons are numbered by type), consecutive positions give some
  //    workgroups several times the mean work; then the rows and pieces are dealt out instead.  Sorted longest first
  //    (stable), they are cut into units of 8 consecutive ones, a slot's worth of like length; each unit goes to the
  //    wave with the least work that has room for a whole unit, and the rows left over once no unit fits go one by
  //    one to the wave with the least work that has a free position (ties: the lower wave).  Every wave's work is
  //    then close to the mean whatever its number of positions, and its slots hold rows of like length (dealt one
  //    row at a time, every wave would get one row from each length and its slots would run to their longest).  A
  //    layout within 5% of the mean is kept (cfg.deal: 1 deals always, -1 never).
  {
    std::vector<int64_t> vlen((size_t)(nrows + t->pieces));
    for (int64_t r = 0; r < nrows; ++r) vlen[r] = rp[r + 1] - rp[r];
    for (int64_t q = 0; q < t->pieces; ++q) {
      const PieceDesc &d = pieces[q];
      const int64_t len = rp[d.row + 1] - rp[d.row];
      vlen[nrows + q] = len * (d.index + 1) / d.count - len * d.index / d.count;
    }
    const int64_t wg_pos = 16 * per, n_wg = (t->npos + wg_pos - 1) / wg_pos;
    std::vector<int64_t> tot((size_t)n_wg, 0);
    int64_t all = 0;
    for (int64_t p = 0; p < t->npos; ++p) {
      tot[p / wg_pos] += vlen[ord[p]];
      all += vlen[ord[p]];
    }
    const int64_t mx = *std::max_element(tot.begin(), tot.end());
    if (cfg.deal > 0 || (cfg.deal == 0 && mx * 20 * n_wg > all * 21)) {
      std::vector<int32_t> items(ord);
      std::stable_sort(items.begin(), items.end(), [&](int32_t a, int32_t b) { return vlen[a] > vlen[b]; });
      typedef std::pair<int64_t, int64_t> Bin;   // (work, wave)
      std::vector<std::vector<int32_t>> bins((size_t)segs);
      std::vector<int64_t> cap((size_t)segs), work((size_t)segs, 0);
      int64_t units = 0;
      for (int64_t w = 0; w < segs; ++w) {
        cap[w] = std::min(per, t->npos - w * per);
        units += cap[w] / 8;
      }
      {  // whole units
        std::priority_queue<Bin, std::vector<Bin>, std::greater<Bin>> heap;
        for (int64_t w = 0; w < segs; ++w)
          if (cap[w] >= 8) heap.push({0, w});
        for (int64_t u = 0; u < units; ++u) {
          const Bin top = heap.top();
          heap.pop();
          const int64_t w = top.second;
          int64_t sum = 0;
          for (int64_t k = 8 * u; k < 8 * u + 8; ++k) {
            bins[w].push_back(items[k]);
            sum += vlen[items[k]];
          }
          work[w] = top.first + sum;
          if ((int64_t)bins[w].size() + 8 <= cap[w]) heap.push({work[w], w});
        }
      }
      {  // the rest, one by one
        std::priority_queue<Bin, std::vector<Bin>, std::greater<Bin>> heap;
        for (int64_t w = 0; w < segs; ++w)
          if ((int64_t)bins[w].size() < cap[w]) heap.push({work[w], w});
        for (size_t k = (size_t)(8 * units); k < items.size(); ++k) {
          const Bin top = heap.top();
          heap.pop();
          const int64_t w = top.second;
          bins[w].push_back(items[k]);
          work[w] = top.first + vlen[items[k]];
          if ((int64_t)bins[w].size() < cap[w]) heap.push({work[w], w});
        }
      }
      for (int64_t w = 0; w < segs; ++w)
        for (size_t k = 0; k < bins[w].size(); ++k) ord[w * per + (int64_t)k] = bins[w][k];
      t->dealt = 1;
    }
  }
  t->rows_per_wave = (int32_t)per;
  t->order.alloc((size_t)t->npos);
  // the float32 kernel walks pairs of slots in one pass when a wave owns over 24 rows (launch_swept)
  t->paired = cfg.paired && K == 4 && per > 24 ? 1 : 0;
  if (!cfg.search) {
    FLY_HIP(hipMemcpyAsync(t->order.p, ord.data(), sizeof(int32_t) * ord.size(), hipMemcpyHostToDevice, st));
  } else {
    DevArray<int32_t> init((size_t)t->npos);
    FLY_HIP(hipMemcpyAsync(init.p, ord.data(), sizeof(int32_t) * ord.size(), hipMemcpyHostToDevice, st));
    if (per <= 4096)
      hipLaunchKernelGGL(k_sweep_order_lds, dim3((unsigned)segs), dim3(64), (unsigned)(per * sizeof(int32_t)), st,
                         t->range.p, K, init.p, t->npos, per, t->order.p);
    else
      hipLaunchKernelGGL(k_sweep_order, dim3(blocks_for(segs, 64)), dim3(64), 0, st, t->range.p, K, init.p, t->npos,
                         per, t->order.p);
    if (per <= kSearchRows) {
      hipLaunchKernelGGL(k_sweep_order_search, dim3((unsigned)segs), dim3(64), 0, st, t->range.p, K, t->npos, per,
                         (int)t->paired, t->order.p);
      hipLaunchKernelGGL(k_sweep_order_balance, dim3((unsigned)((segs + 15) / 16)), dim3(kBalanceThreads), 0, st,
                         t->range.p, K, t->npos, per, (int)t->paired, t->order.p);
    }
    check_launch("sweep order");
    FLY_HIP(hipStreamSynchronize(st));
  }
  FLY_HIP(hipStreamSynchronize(st));
  return t;
}

// The configuration of a plan's or fly_sweep's tables from its tuning (the order is searched for passes of two
// slots when the tuning makes the sweep walk them).
inline SweepConfig sweep_config(const Tuning &tu) {
  SweepConfig c;
  c.bands = tu.sweep_bands == 3 ? 3 : kSweepBands;
  c.paired = tu.sweep_paired > 0 ? 1 : 0;
  c.grid = tu.sweep_grid > 0 ? tu.sweep_grid : 0;
  c.force = tu.swept > 0 ? 1 : 0;
  c.piece = tu.sweep_piece > 0 ? tu.sweep_piece : 0;
  c.search = tu.sweep_order >= 0 ? 1 : 0;
  c.deal = tu.sweep_deal > 0 ? 1 : (tu.sweep_deal < 0 ? -1 : 0);
  return c;
}

struct ConeSweepCache {
  struct Entry {
    int t;
    SweepConfig cfg;
    std::shared_ptr<const SweepTables> tables;   // null: the step does not sweep under cfg
  };
  std::mutex mu;
  std::vector<Entry> entries;
};

}  // namespace fly
