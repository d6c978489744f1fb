// Dense maps of the network on the matrix cores, and the whole-model forward.
//
//   encoder  u[m, b] = (sum_k W[m, k] x[b, k] + bias[m]) * gain              chessfly/model.py:99-102
//   head     r[b, j] = clamp((c_base[j] + X_T[src_j, b] - mean_j) / sqrt(var_j + eps), -clip, clip)
//            logits[b, i] = (P r + bp)[i] + (F r + bf)[from_i] + (T r + bt)[to_i],  wdl = V r + bv
//                                                                            chessfly/model.py:51-58, 103-105
// float32 accuracy on fp16 matrix cores: every operand is split into hi = fp16(v) and lo = fp16(v - hi) (22
// significant bits together) and C = A_hi B_hi + A_hi B_lo + A_lo B_hi is accumulated in float32 with
// v_mfma_f32_16x16x32_f16 (the dropped A_lo B_lo term is below float32 round-off).  Weights are scaled by a
// power of two before the split so their low parts stay clear of fp16 subnormals; the scale is undone
// exactly on the accumulator.  The weights are split once per weight version into a dense plan (fly_dense);
// the boards and the normalised outputs are split per forward by small prologue kernels, the latter reading
// the final recurrent state in place (output gather, normaliser and transpose in one pass).
//
// GEMM tiling: C = A B^T with both operands K-contiguous (K padded to 64 with zeros).  A workgroup of 4 waves
// owns a 128 x 128, 128 x 64 or 64 x 64 output tile (2 x 2 waves, each a grid of 16 x 16 MFMA tiles); K is staged 64
// at a time through LDS as hi/lo halves with the next stage's 16-byte global loads in flight, and tiles are
// ordered so the workgroups one XCD runs together share operand rows in its L2.  The boards' lo half is zero when
// they are exact in float16 (binary planes always are); the split records that per board and a tile whose boards
// are all exact leaves out the A_hi B_lo product.
#include "common.hpp"

#include <cmath>
#include <cstring>
#include <mutex>
#include <string>

namespace fly {

int64_t io_block(const fly_plan &plan, int64_t batch);
size_t io_workspace(const fly_plan &plan, int64_t batch);
size_t plan_pieces_bytes(const fly_plan &plan, int64_t batch);
template <typename S, typename U>
const S *run_cone_steps(const fly_plan &plan, const U *u, int64_t ldu, int64_t batch, bool u_padded, void *ws,
                        float *pieces, hipStream_t st);
void check_plan_device(const fly_plan *plan);

}  // namespace fly

struct fly_dense {
  int device = -1;
  int64_t n_in = 0, k = 0, kp_enc = 0;            // encoder: n_in rows over k feature columns (padded to kp_enc)
  int64_t n_out = 0, n_moves = 0, kp_head = 0;    // head: n_moves + 131 rows over n_out outputs
  fly::DevArray<_Float16> enc_hi, enc_lo, head_hi, head_lo;
  fly::DevArray<float> enc_b, head_b, norm_mean, norm_var;
  fly::DevArray<int32_t> move_from, move_to;
  float enc_unscale = 1.f, head_unscale = 1.f, eps = 1e-8f, clip = 8.f;
  int gemm_tile = 0;   // the gemm_tile tuning when the dense plan was created
  int64_t head_rows() const { return n_moves + 131; }
};

namespace fly {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int GBK = 64, LDK = GBK + 8;  // K per LDS stage; LDS rows padded to 144 bytes

int64_t pad_k(int64_t k) { return round_up(std::max<int64_t>(k, 1), GBK); }

// hi = fp16(v * scale), lo = fp16(v * scale - hi), rows x kp, zero beyond k; one workgroup per row.  A float16
// source widens exactly, so with scale 1 its lo half is zero.  flag[r] (when given) records whether any lo of row r
// is non-zero, so the GEMM can leave out the product with a tile's lo half when every row of the tile is exact.
template <typename T>
__global__ __launch_bounds__(256) void k_split_rows(const T *__restrict__ src, int64_t ld, int64_t k, float scale,
                                                    _Float16 *__restrict__ hi, _Float16 *__restrict__ lo, int64_t kp,
                                                    int32_t *__restrict__ flag) {
  const int64_t r = blockIdx.x;
  bool any = false;
  for (int64_t c = threadIdx.x; c < kp; c += blockDim.x) {
    const float v = c < k ? static_cast<float>(src[r * ld + c]) * scale : 0.0f;
    const _Float16 h = static_cast<_Float16>(v);
    const _Float16 l = static_cast<_Float16>(v - static_cast<float>(h));
    hi[r * kp + c] = h;
    lo[r * kp + c] = l;
    any |= l != static_cast<_Float16>(0.0f);
  }
  if (flag != nullptr) {
    const int a = __syncthreads_or(any);
    if (threadIdx.x == 0) flag[r] = a;
  }
}

// Normalised outputs r[n, k] split into (N x kp) hi/lo rows, read from the state (rows, lds) where output k
// sits at row src[k] (-1: not carried; src null: row k), plus cbase[k] (null: 0).  A 64x64 tile goes through
// LDS so both the state reads (n fastest) and the split writes (k fastest) are contiguous; each thread reads 4
// boards of a row (one 8- or 16-byte load when `vec`: the state's rows hold whole groups of 4) and writes 4
// outputs of a board (8-byte stores of hi and lo).
template <typename S>
__global__ __launch_bounds__(256) void k_norm_split(const S *__restrict__ state, int64_t lds, bool vec,
                                                    const int32_t *__restrict__ src, const float *__restrict__ cbase,
                                                    const float *__restrict__ mean, const float *__restrict__ var,
                                                    float eps, float clip, int64_t K, int64_t N,
                                                    _Float16 *__restrict__ hi, _Float16 *__restrict__ lo, int64_t kp) {
  typedef S vec4 __attribute__((ext_vector_type(4)));
  typedef _Float16 half4 __attribute__((ext_vector_type(4)));
  __shared__ float tile[64][65];
  const int64_t k0 = (int64_t)blockIdx.y * 64, n0 = (int64_t)blockIdx.x * 64;
  const int q = (threadIdx.x & 15) * 4, r16 = threadIdx.x >> 4;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int kk = r16 + 16 * j;
    const int64_t k = k0 + kk, n = n0 + q;
    float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (k < K) {
      const int32_t row = src ? src[k] : (int32_t)k;
      const float c = cbase ? cbase[k] : 0.0f, m = mean[k], sd = sqrtf(var[k] + eps);
      float x[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      if (state != nullptr && row >= 0) {
        const S *p = state + (int64_t)row * lds + n;
        if (vec && n + 3 < N) {
          const vec4 w = *reinterpret_cast<const vec4 *>(p);
#pragma unroll
          for (int i = 0; i < 4; ++i) x[i] = static_cast<float>(w[i]);
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i) x[i] = n + i < N ? static_cast<float>(p[i]) : 0.0f;
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (n + i < N) v[i] = fminf(fmaxf(((c + x[i]) - m) / sd, -clip), clip);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) tile[kk][q + i] = v[i];
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int nn = r16 + 16 * j;
    const int64_t n = n0 + nn, k = k0 + q;
    if (n < N && k < kp) {   // kp is a multiple of 64: the 4 outputs are inside the row
      half4 h, l;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float v = tile[q + i][nn];
        h[i] = static_cast<_Float16>(v);
        l[i] = static_cast<_Float16>(v - static_cast<float>(h[i]));
      }
      *reinterpret_cast<half4 *>(hi + n * kp + k) = h;
      *reinterpret_cast<half4 *>(lo + n * kp + k) = l;
    }
  }
}

struct Split {
  const _Float16 *hi, *lo;
  int64_t rows;          // leading dimension is the padded K
  const int32_t *flag;   // per row: lo is non-zero somewhere (null: assume it is)
};

// u[m, n] = (C[m, n] + bias[m]) * gain.  The tile is staged through LDS and written as whole rows (kRows):
// per element, a wave's stores covered four 64-byte pieces of four rows, and the encoder's 80 MB output took a
// quarter of its time.
struct EncoderEpilogue {
  static constexpr bool kRows = true;
  const float *bias;
  float gain;
  float *u;
  _Float16 *u16;
  int64_t ldu;
  __device__ __forceinline__ void operator()(int64_t m, int64_t n, float v) const {
    const float x = (v + bias[m]) * gain;
    if (u16) u16[m * ldu + n] = static_cast<_Float16>(x);
    else u[m * ldu + n] = x;
  }
  // columns n .. n + 3 of row m (avail of them inside the output); 16-byte stores when the row allows them
  __device__ __forceinline__ void row4(int64_t m, int64_t n, float4 v, int64_t avail) const {
    const float b = bias[m];
    const float x[4] = {(v.x + b) * gain, (v.y + b) * gain, (v.z + b) * gain, (v.w + b) * gain};
    if (!u16 && avail >= 4 && (reinterpret_cast<uintptr_t>(u + m * ldu + n) & 15) == 0) {
      *reinterpret_cast<float4 *>(u + m * ldu + n) = make_float4(x[0], x[1], x[2], x[3]);
      return;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (i < avail) {
        if (u16) u16[m * ldu + n + i] = static_cast<_Float16>(x[i]);
        else u[m * ldu + n + i] = x[i];
      }
  }
};

// ct[n, m] = C[m, n]: one row of all head outputs per board (measured: its element stores cost about 4 us).
struct HeadEpilogue {
  static constexpr bool kRows = false;
  float *ct;
  int64_t ldc;
  __device__ __forceinline__ void operator()(int64_t m, int64_t n, float v) const { ct[n * ldc + m] = v; }
  __device__ __forceinline__ void row4(int64_t, int64_t, float4, int64_t) const {}
};

__device__ __forceinline__ half8 load8(const _Float16 *p) { return *reinterpret_cast<const half8 *>(p); }

// Tile order: the dispatcher hands workgroup L to XCD L mod 8, so the tile of workgroup L is chosen to give each
// XCD a contiguous run of tiles in row-major (A-tile, B-tile) order.  The tiles an XCD runs together then share
// their A rows and sweep the same B rows, and each operand crosses into an XCD's L2 about once.
__device__ __forceinline__ void xcd_tile(int tiles, int gx, int &ty, int &tx) {
  const int L = blockIdx.x, xcd = L & 7, slot = L >> 3, per = tiles >> 3, rem = tiles & 7;
  const int q = xcd * per + min(xcd, rem) + slot;
  ty = q / gx;
  tx = q - ty * gx;
}

// C = A B^T on split operands.  4 waves in 2 x 2, each owning (16 TM) x (16 TN) of the (32 TM) x (32 TN) tile.
// K is staged 64 at a time through LDS: each row of a stage is one 128-byte line, loaded by 8 consecutive lanes and
// written to LDS in one piece; rows are padded to 144 bytes so 16-byte fragment reads are free of bank conflicts.  The
// next stage's global loads are issued before the current stage's MFMAs.  BLO = false leaves out A_hi B_lo, for tiles
// whose B rows are all exact in float16.
template <int TM, int TN, bool BLO, class EP>
__device__ __forceinline__ void gemm_tile(const Split &A, const Split &B, int64_t kp, float unscale, const EP &ep,
                                          int64_t m0, int64_t n0, _Float16 (*As)[32 * TM][LDK],
                                          _Float16 (*Bs)[32 * TN][LDK]) {
  constexpr int OCT = GBK / 8, RPP = 256 / OCT;          // 16-byte pieces per row, rows per pass of 256 threads
  constexpr int AL = 32 * TM / RPP, BL = 32 * TN / RPP;  // passes per operand half
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int lr = tid / OCT, lk = (tid % OCT) * 8;  // one full 128-byte line of K per row and stage
  const half8 zero = {0, 0, 0, 0, 0, 0, 0, 0};
  int64_t aoff[AL], boff[BL];
  bool aok[AL], bok[BL];
#pragma unroll
  for (int i = 0; i < AL; ++i) {
    aok[i] = m0 + lr + RPP * i < A.rows;
    aoff[i] = (aok[i] ? m0 + lr + RPP * i : 0) * kp + lk;
  }
#pragma unroll
  for (int i = 0; i < BL; ++i) {
    bok[i] = n0 + lr + RPP * i < B.rows;
    boff[i] = (bok[i] ? n0 + lr + RPP * i : 0) * kp + lk;
  }
  half8 rah[AL], ral[AL], rbh[BL], rbl[BL];
  auto fetch = [&](int64_t k0) {
#pragma unroll
    for (int i = 0; i < AL; ++i) {
      rah[i] = aok[i] ? load8(A.hi + aoff[i] + k0) : zero;
      ral[i] = aok[i] ? load8(A.lo + aoff[i] + k0) : zero;
    }
#pragma unroll
    for (int i = 0; i < BL; ++i) {
      rbh[i] = bok[i] ? load8(B.hi + boff[i] + k0) : zero;
      if (BLO) rbl[i] = bok[i] ? load8(B.lo + boff[i] + k0) : zero;
    }
  };
  floatx4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
  const int fk = 8 * (lane >> 4), fr = lane & 15;
  fetch(0);
  for (int64_t k0 = 0; k0 < kp; k0 += GBK) {
#pragma unroll
    for (int i = 0; i < AL; ++i) {
      *reinterpret_cast<half8 *>(&As[0][lr + RPP * i][lk]) = rah[i];
      *reinterpret_cast<half8 *>(&As[1][lr + RPP * i][lk]) = ral[i];
    }
#pragma unroll
    for (int i = 0; i < BL; ++i) {
      *reinterpret_cast<half8 *>(&Bs[0][lr + RPP * i][lk]) = rbh[i];
      if (BLO) *reinterpret_cast<half8 *>(&Bs[1][lr + RPP * i][lk]) = rbl[i];
    }
    __syncthreads();
    if (k0 + GBK < kp) fetch(k0 + GBK);
#pragma unroll
    for (int kk = 0; kk < GBK; kk += 32) {
      half8 bh[TN], bl[TN];
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        bh[j] = *reinterpret_cast<const half8 *>(&Bs[0][wn * 16 * TN + j * 16 + fr][kk + fk]);
        if (BLO) bl[j] = *reinterpret_cast<const half8 *>(&Bs[1][wn * 16 * TN + j * 16 + fr][kk + fk]);
      }
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const half8 ah = *reinterpret_cast<const half8 *>(&As[0][wm * 16 * TM + i * 16 + fr][kk + fk]);
        const half8 al = *reinterpret_cast<const half8 *>(&As[1][wm * 16 * TM + i * 16 + fr][kk + fk]);
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bh[j], acc[i][j], 0, 0, 0);
          if (BLO) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bl[j], acc[i][j], 0, 0, 0);
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bh[j], acc[i][j], 0, 0, 0);
        }
      }
    }
    __syncthreads();
  }
  if constexpr (EP::kRows) {
    // The operand stages are free after the last barrier: C goes through them, rows padded by 4 floats, and
    // leaves as 16-byte pieces of whole rows (a wave writes two 512-byte rows per store at 128 columns).
    constexpr int LDC = 32 * TN + 4, V4 = 32 * TN / 4;
    float *Cs = reinterpret_cast<float *>(&As[0][0][0]);   // k_gemm_split sizes its LDS for the C tile too
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          Cs[(wm * 16 * TM + i * 16 + 4 * (lane >> 4) + r) * LDC + wn * 16 * TN + j * 16 + (lane & 15)] =
              acc[i][j][r] * unscale;
    __syncthreads();
    for (int idx = tid; idx < 32 * TM * V4; idx += 256) {
      const int rr = idx / V4, c4 = idx - rr * V4;
      const int64_t m = m0 + rr, n = n0 + 4 * c4;
      if (m < A.rows && n < B.rows)
        ep.row4(m, n, *reinterpret_cast<const float4 *>(&Cs[rr * LDC + 4 * c4]), B.rows - n);
    }
  } else {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int64_t m = m0 + wm * 16 * TM + i * 16 + 4 * (lane >> 4) + r;
          const int64_t n = n0 + wn * 16 * TN + j * 16 + (lane & 15);
          if (m < A.rows && n < B.rows) ep(m, n, acc[i][j][r] * unscale);
        }
  }
}

template <int TM, int TN, class EP>
__global__ __launch_bounds__(256) void k_gemm_split(const Split A, const Split B, int64_t kp, float unscale, const EP ep,
                                                    int tiles, int gx) {
  // one block of LDS for both operands' stages and, after the K loop, the C tile of a row-wise epilogue (rows
  // padded by 4 floats)
  constexpr size_t kStages = 2 * LDK * 32 * (TM + TN);
  constexpr size_t kCTile = EP::kRows ? (size_t)32 * TM * (32 * TN + 4) * 2 : 0;   // in halves
  __shared__ __attribute__((aligned(16))) _Float16 smem[kStages > kCTile ? kStages : kCTile];
  auto As = reinterpret_cast<_Float16 (*)[32 * TM][LDK]>(smem);
  auto Bs = reinterpret_cast<_Float16 (*)[32 * TN][LDK]>(smem + 2 * LDK * 32 * TM);
  int ty, tx;
  xcd_tile(tiles, gx, ty, tx);
  const int64_t m0 = (int64_t)ty * (32 * TM), n0 = (int64_t)tx * (32 * TN);
  bool blo = true;
  if (B.flag != nullptr) {  // uniform over the workgroup
    const int i = threadIdx.x;
    blo = __syncthreads_or(i < 32 * TN && n0 + i < B.rows && B.flag[n0 + i] != 0);
  }
  if (blo)
    gemm_tile<TM, TN, true>(A, B, kp, unscale, ep, m0, n0, As, Bs);
  else
    gemm_tile<TM, TN, false>(A, B, kp, unscale, ep, m0, n0, As, Bs);
}

// Wave tiles of 64 x 64 (128 x 128 per workgroup) where that gives at least four tiles per CU, else 32 x 32 or
// 32 x 80 (64 x 64 or 64 x 160 per workgroup): measured on the 17,937 x 1120 encoder and the 4,299 x 1120 head.
// The gemm_tile tuning key forces one: 1 = 64 x 64, 2 = 128 x 64, 3 = 128 x 128, or 10 TM + TN for a workgroup tile
// of 32 TM x 32 TN with TM in {2, 3, 4} and TN in {2, 4, 5}.
template <class EP>
void gemm_split(const Split &A, const Split &B, int64_t kp, float unscale, const EP &ep, int tile_key,
                hipStream_t st) {
  if (A.rows == 0 || B.rows == 0) return;
  auto count = [&](int bm, int bn) { return ((A.rows + bm - 1) / bm) * ((B.rows + bn - 1) / bn); };
  int shape = tile_key;
  if (shape == 1) shape = 22;
  else if (shape == 2) shape = 42;
  else if (shape == 3) shape = 44;
  const int tm = shape / 10, tn = shape % 10;
  const bool known = (tm == 2 || tm == 3 || tm == 4) && (tn == 2 || tn == 4 || tn == 5);
  // smaller GEMMs (the head): 64 x 160 where 160-column tiles cover the batch with no more padding than 64-column
  // ones (B = 1120: 7 tiles against 17.5, one round of workgroups; 6 us faster), else 64 x 64
  if (!known) shape = count(128, 128) >= 1024 ? 44 : (round_up(B.rows, 160) <= round_up(B.rows, 64) ? 25 : 22);
  const int bm = 32 * (shape / 10), bn = 32 * (shape % 10);
  const int64_t gx = (B.rows + bn - 1) / bn, tiles = count(bm, bn);
  FLY_REQUIRE(tiles < INT32_MAX, "GEMM grid too large");
  const dim3 grid((unsigned)tiles), block(256);
#define FLY_GEMM_CASE(TM_, TN_)                                                                                    \
  case 10 * TM_ + TN_:                                                                                             \
    hipLaunchKernelGGL((k_gemm_split<TM_, TN_, EP>), grid, block, 0, st, A, B, kp, unscale, ep, (int)tiles, (int)gx); \
    break;
  switch (shape) {
    FLY_GEMM_CASE(2, 2)
    FLY_GEMM_CASE(2, 4)
    FLY_GEMM_CASE(2, 5)
    FLY_GEMM_CASE(3, 2)
    FLY_GEMM_CASE(3, 4)
    FLY_GEMM_CASE(3, 5)
    FLY_GEMM_CASE(4, 2)
    FLY_GEMM_CASE(4, 4)
    FLY_GEMM_CASE(4, 5)
    default: FLY_REQUIRE(false, "unknown GEMM tile");
  }
#undef FLY_GEMM_CASE
  check_launch("split gemm");
}

// logits[n, i] = (ct[n, i] + b[i]) + (ct[n, M + f] + b[M + f]) + (ct[n, M + 64 + t] + b[M + 64 + t]),
// wdl[n, j] = ct[n, M + 128 + j] + b[M + 128 + j], with M = n_moves and (f, t) the move's squares.
// One workgroup per board: its from- and to-square terms (64 + 64 values plus biases) go to LDS once, then each
// thread writes 4 consecutive moves with 16-byte loads and stores when `vec` (the move count and the rows allow
// them), one move at a time otherwise.
__global__ __launch_bounds__(256) void k_assemble(const float *__restrict__ ct, int64_t ldc, int64_t n_moves,
                                                  const float *__restrict__ b, const int32_t *__restrict__ mfrom,
                                                  const int32_t *__restrict__ mto, int64_t batch, bool vec,
                                                  float *__restrict__ logits, float *__restrict__ wdl) {
  __shared__ float sq[128];
  for (int64_t n = blockIdx.x; n < batch; n += gridDim.x) {
    const float *row = ct + n * ldc;
    __syncthreads();   // the previous board's squares are read
    if (threadIdx.x < 128) sq[threadIdx.x] = row[n_moves + threadIdx.x] + b[n_moves + threadIdx.x];
    if (threadIdx.x < 3) wdl[n * 3 + threadIdx.x] = row[n_moves + 128 + threadIdx.x] + b[n_moves + 128 + threadIdx.x];
    __syncthreads();
    float *out = logits + n * n_moves;
    if (vec) {
      for (int64_t i = 4 * (int64_t)threadIdx.x; i < n_moves; i += 4 * (int64_t)blockDim.x) {
        const float4 p = *reinterpret_cast<const float4 *>(row + i), bp = *reinterpret_cast<const float4 *>(b + i);
        const int4 fr = *reinterpret_cast<const int4 *>(mfrom + i), to = *reinterpret_cast<const int4 *>(mto + i);
        *reinterpret_cast<float4 *>(out + i) =
            make_float4(((p.x + bp.x) + sq[fr.x]) + sq[64 + to.x], ((p.y + bp.y) + sq[fr.y]) + sq[64 + to.y],
                        ((p.z + bp.z) + sq[fr.z]) + sq[64 + to.z], ((p.w + bp.w) + sq[fr.w]) + sq[64 + to.w]);
      }
    } else {
      for (int64_t i = threadIdx.x; i < n_moves; i += blockDim.x)
        out[i] = ((row[i] + b[i]) + sq[mfrom[i]]) + sq[64 + mto[i]];
    }
  }
}

// Grid-stride max of |w| with one atomic per wave (a fixed grid keeps the atomics on the one word few).
__global__ void k_max_abs(const float *__restrict__ w, int64_t ld, int64_t rows, int64_t k, unsigned *__restrict__ out) {
  float a = 0.0f;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < rows * k; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / k, c = i - r * k;
    a = fmaxf(a, fabsf(w[r * ld + c]));
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) a = fmaxf(a, __shfl_xor(a, off));
  // non-negative floats order like their bit patterns
  if ((threadIdx.x & 63) == 0 && a > 0.0f) atomicMax(out, __float_as_uint(a));
}

__global__ void k_check_squares(const int32_t *__restrict__ sq, int64_t n, int32_t *__restrict__ bad) {
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i < n && (sq[i] < 0 || sq[i] > 63)) atomicOr(bad, 1);
}

__global__ void k_zero_u32(unsigned *__restrict__ p) { *p = 0u; }

constexpr int kThreads = 256;

// Power-of-two scale that puts the largest |w| at 2^14 (low halves stay normal fp16 for every weight that
// matters); 1 for an all-zero matrix.
float weight_scale(const float *w, int64_t ld, int64_t rows, int64_t k, hipStream_t st) {
  if (rows * k == 0) return 1.0f;
  DevArray<unsigned> mx(1);
  hipLaunchKernelGGL(k_zero_u32, dim3(1), dim3(1), 0, st, mx.p);
  hipLaunchKernelGGL(k_max_abs, dim3((unsigned)std::min<int64_t>(blocks_for(rows * k, kThreads), 1024)), dim3(kThreads), 0,
                     st, w, ld, rows, k, mx.p);
  check_launch("max abs");
  unsigned bits = 0;
  FLY_HIP(hipMemcpyAsync(&bits, mx.p, sizeof(bits), hipMemcpyDeviceToHost, st));
  FLY_HIP(hipStreamSynchronize(st));
  float m;
  memcpy(&m, &bits, sizeof(m));
  FLY_REQUIRE(std::isfinite(m), "dense weights hold a non-finite value");
  if (m == 0.0f) return 1.0f;
  const int e = std::max(-24, std::min(24, 14 - (int)std::ceil(std::log2(m))));
  return std::ldexp(1.0f, e);
}

template <typename T>
void split_into(const T *w, int64_t ld, int64_t rows, int64_t k, float scale, _Float16 *hi, _Float16 *lo,
                int64_t kp, hipStream_t st, int32_t *flag = nullptr) {
  if (rows == 0) return;
  FLY_REQUIRE(rows < INT32_MAX, "too many rows to split");
  hipLaunchKernelGGL(k_split_rows<T>, dim3((unsigned)rows), dim3(kThreads), 0, st, w, ld, k, scale, hi, lo, kp, flag);
  check_launch("split");
}


int64_t head_ld(const fly_dense &d) { return round_up(d.head_rows(), 4); }

size_t split_bytes(int64_t rows, int64_t kp) { return align256((size_t)rows * kp * sizeof(_Float16)); }

size_t encoder_ws(const fly_dense &d, int64_t batch) {
  return 2 * split_bytes(batch, d.kp_enc) + align256((size_t)batch * sizeof(int32_t));
}

size_t head_ws(const fly_dense &d, int64_t batch) {
  return 2 * split_bytes(batch, d.kp_head) + align256((size_t)batch * head_ld(d) * sizeof(float));
}

void run_encoder(const fly_dense &d, const void *x, bool x_f16, int64_t ldx, int64_t batch, float gain, float *u,
                 _Float16 *u16, int64_t ldu, void *ws, hipStream_t st) {
  LaunchTimer timer(FLY_K_ENCODER, st);
  _Float16 *xh = static_cast<_Float16 *>(ws);
  _Float16 *xl = reinterpret_cast<_Float16 *>(static_cast<char *>(ws) + split_bytes(batch, d.kp_enc));
  int32_t *exact = reinterpret_cast<int32_t *>(static_cast<char *>(ws) + 2 * split_bytes(batch, d.kp_enc));
  if (x_f16)
    split_into(static_cast<const _Float16 *>(x), ldx, batch, d.k, 1.0f, xh, xl, d.kp_enc, st, exact);
  else
    split_into(static_cast<const float *>(x), ldx, batch, d.k, 1.0f, xh, xl, d.kp_enc, st, exact);
  gemm_split(Split{d.enc_hi.p, d.enc_lo.p, d.n_in, nullptr}, Split{xh, xl, batch, exact}, d.kp_enc, d.enc_unscale,
             EncoderEpilogue{d.enc_b.p, gain, u, u16, ldu}, d.gemm_tile, st);
}

template <typename S>
void run_head(const fly_dense &d, const S *state, int64_t lds, const int32_t *src, const float *cbase, int64_t batch,
              float *logits, float *wdl, void *ws, hipStream_t st) {
  LaunchTimer timer(FLY_K_HEAD, st);
  char *base = static_cast<char *>(ws);
  _Float16 *rh = reinterpret_cast<_Float16 *>(base);
  _Float16 *rl = reinterpret_cast<_Float16 *>(base + split_bytes(batch, d.kp_head));
  float *ct = reinterpret_cast<float *>(base + 2 * split_bytes(batch, d.kp_head));
  const dim3 grid(blocks_for(batch, 64), (unsigned)((d.kp_head + 63) / 64));
  const bool vec = lds % 4 == 0 && aligned(state, 4 * sizeof(S));
  hipLaunchKernelGGL(k_norm_split<S>, grid, dim3(256), 0, st, state, lds, vec, src, cbase, d.norm_mean.p, d.norm_var.p,
                     d.eps, d.clip, d.n_out, batch, rh, rl, d.kp_head);
  check_launch("normalised outputs");
  const int64_t ldc = head_ld(d);
  gemm_split(Split{d.head_hi.p, d.head_lo.p, d.head_rows(), nullptr}, Split{rh, rl, batch, nullptr}, d.kp_head,
             d.head_unscale,
             HeadEpilogue{ct, ldc}, d.gemm_tile, st);
  const bool avec = d.n_moves % 4 == 0 && ldc % 4 == 0 && aligned(logits, 16);
  hipLaunchKernelGGL(k_assemble, dim3((unsigned)std::min<int64_t>(batch, 65535)), dim3(256), 0, st, ct, ldc, d.n_moves,
                     d.head_b.p, d.move_from.p, d.move_to.p, batch, avec, logits, wdl);
  check_launch("head assembly");
}

void check_dense(const fly_dense *d) {
  FLY_REQUIRE(d != nullptr, "dense plan is null");
  FLY_REQUIRE(current_device() == d->device, "the dense plan lives on another device");
}

}  // namespace
}  // namespace fly

using namespace fly;

extern "C" int fly_dense_create(const fly_head_desc *h, const float *enc_w, int64_t ldw, int64_t k,
                                const float *enc_b, int64_t n_in, void *stream, fly_dense **out) {
  return guard([&] {
    FLY_REQUIRE(out != nullptr, "out is null");
    *out = nullptr;
    FLY_REQUIRE(h != nullptr, "head is null");
    FLY_REQUIRE(h->n_out > 0 && h->n_moves > 0 && n_in >= 0 && k >= 0 && ldw >= k, "bad size");
    FLY_REQUIRE(h->norm_mean && h->norm_var && h->policy_w && h->policy_b && h->from_w && h->from_b && h->to_w &&
                    h->to_b && h->value_w && h->value_b && h->move_from && h->move_to,
                "head has a null pointer");
    FLY_REQUIRE(n_in == 0 || (enc_w && enc_b), "encoder has a null pointer");
    hipStream_t st = as_stream(stream);
    auto d = std::make_unique<fly_dense>();
    d->device = current_device();
    d->gemm_tile = tuning_snapshot().gemm_tile;
    d->n_in = n_in;
    d->k = k;
    d->kp_enc = pad_k(k);
    d->n_out = h->n_out;
    d->n_moves = h->n_moves;
    d->kp_head = pad_k(h->n_out);
    d->eps = h->norm_eps;
    d->clip = h->norm_clip;
    {  // move squares must index the 64 from/to rows
      DevArray<int32_t> bad(1);
      hipLaunchKernelGGL(k_zero_u32, dim3(1), dim3(1), 0, st, reinterpret_cast<unsigned *>(bad.p));
      hipLaunchKernelGGL(k_check_squares, dim3(blocks_for(h->n_moves, kThreads)), dim3(kThreads), 0, st, h->move_from,
                         h->n_moves, bad.p);
      hipLaunchKernelGGL(k_check_squares, dim3(blocks_for(h->n_moves, kThreads)), dim3(kThreads), 0, st, h->move_to,
                         h->n_moves, bad.p);
      check_launch("square check");
      int32_t hb = 0;
      FLY_HIP(hipMemcpyAsync(&hb, bad.p, sizeof(hb), hipMemcpyDeviceToHost, st));
      FLY_HIP(hipStreamSynchronize(st));
      FLY_REQUIRE(hb == 0, "move_from / move_to hold a square outside 0..63");
    }
    // encoder
    const float es = weight_scale(enc_w, ldw, n_in, k, st);
    d->enc_unscale = 1.0f / es;
    d->enc_hi.alloc(n_in * d->kp_enc);
    d->enc_lo.alloc(n_in * d->kp_enc);
    split_into(enc_w, ldw, n_in, k, es, d->enc_hi.p, d->enc_lo.p, d->kp_enc, st);
    d->enc_b.alloc(n_in);
    if (n_in) FLY_HIP(hipMemcpyAsync(d->enc_b.p, enc_b, sizeof(float) * n_in, hipMemcpyDeviceToDevice, st));
    // head: policy, from, to and value rows stacked under one scale
    const int64_t K = h->n_out, M = h->n_moves;
    struct Part {
      const float *w, *b;
      int64_t rows, off;
    } parts[4] = {{h->policy_w, h->policy_b, M, 0}, {h->from_w, h->from_b, 64, M}, {h->to_w, h->to_b, 64, M + 64},
                  {h->value_w, h->value_b, 3, M + 128}};
    float hs = 0.0f;
    for (const Part &p : parts) {
      const float s = weight_scale(p.w, K, p.rows, K, st);
      hs = (hs == 0.0f) ? s : std::min(hs, s);
    }
    d->head_unscale = 1.0f / hs;
    d->head_hi.alloc(d->head_rows() * d->kp_head);
    d->head_lo.alloc(d->head_rows() * d->kp_head);
    d->head_b.alloc(d->head_rows());
    for (const Part &p : parts) {
      split_into(p.w, K, p.rows, K, hs, d->head_hi.p + p.off * d->kp_head, d->head_lo.p + p.off * d->kp_head,
                 d->kp_head, st);
      FLY_HIP(hipMemcpyAsync(d->head_b.p + p.off, p.b, sizeof(float) * p.rows, hipMemcpyDeviceToDevice, st));
    }
    d->move_from.alloc(M);
    d->move_to.alloc(M);
    FLY_HIP(hipMemcpyAsync(d->move_from.p, h->move_from, sizeof(int32_t) * M, hipMemcpyDeviceToDevice, st));
    FLY_HIP(hipMemcpyAsync(d->move_to.p, h->move_to, sizeof(int32_t) * M, hipMemcpyDeviceToDevice, st));
    d->norm_mean.alloc(K);
    d->norm_var.alloc(K);
    FLY_HIP(hipMemcpyAsync(d->norm_mean.p, h->norm_mean, sizeof(float) * K, hipMemcpyDeviceToDevice, st));
    FLY_HIP(hipMemcpyAsync(d->norm_var.p, h->norm_var, sizeof(float) * K, hipMemcpyDeviceToDevice, st));
    FLY_HIP(hipStreamSynchronize(st));
    *out = d.release();
  });
}

extern "C" int fly_dense_destroy(fly_dense *d) {
  return guard([&] { delete d; });
}

extern "C" size_t fly_encoder_workspace(const fly_dense *d, int64_t batch) { return d ? encoder_ws(*d, batch) : 0; }

extern "C" int fly_encoder(const fly_dense *d, const void *x, int32_t x_f16, int64_t ldx, int64_t batch, float gain,
                           void *u, int64_t ldu, int32_t out_f16, void *ws, size_t ws_bytes, void *stream) {
  return guard([&] {
    check_dense(d);
    FLY_REQUIRE(batch >= 0, "negative batch");
    if (!batch || !d->n_in) return;
    FLY_REQUIRE(x && u && ldx >= d->k && ldu >= batch, "bad argument");
    FLY_REQUIRE(ws && ws_bytes >= encoder_ws(*d, batch) && aligned(ws, 256), "workspace too small or misaligned");
    run_encoder(*d, x, x_f16 != 0, ldx, batch, gain, out_f16 ? nullptr : static_cast<float *>(u),
                out_f16 ? static_cast<_Float16 *>(u) : nullptr, ldu, ws, as_stream(stream));
  });
}

extern "C" size_t fly_head_workspace(const fly_dense *d, int64_t batch) { return d ? head_ws(*d, batch) : 0; }

extern "C" int fly_head(const fly_dense *d, const float *r, int64_t ldr, int64_t batch, float *logits, float *wdl,
                        void *ws, size_t ws_bytes, void *stream) {
  return guard([&] {
    check_dense(d);
    FLY_REQUIRE(batch >= 0, "negative batch");
    if (!batch) return;
    FLY_REQUIRE(r && ldr >= batch && logits && wdl, "bad argument");
    FLY_REQUIRE(ws && ws_bytes >= head_ws(*d, batch) && aligned(ws, 256), "workspace too small or misaligned");
    run_head<float>(*d, r, ldr, nullptr, nullptr, batch, logits, wdl, ws, as_stream(stream));
  });
}

namespace fly {
namespace {

// Scratch of one block of `blk` boards of the model forward: the encoder's output u (float32, padded rows), the
// two state buffers, then the encoder's operand split or the head's (they never live at once).
size_t model_ws_block(const fly_plan &plan, const fly_dense &d, int64_t blk) {
  const size_t es = plan.mode == FLY_MODE_DEVIATION_F16 ? sizeof(_Float16) : sizeof(float);
  return align256((size_t)plan.n_in * state_ld(blk, sizeof(float)) * sizeof(float)) +
         align256(2 * (size_t)plan.max_rows * (size_t)state_ld(blk, es) * es + 256) + plan_pieces_bytes(plan, blk) +
         std::max(encoder_ws(d, blk), head_ws(d, blk));
}

void check_model_args(const fly_plan *plan, const fly_dense *d, const void *x, int64_t ldx, int64_t batch,
                      const float *logits, const float *wdl) {
  check_plan_device(plan);
  check_dense(d);
  FLY_REQUIRE(!plan->full, "the model forward needs a light-cone plan");
  FLY_REQUIRE(d->n_out == plan->n_out && d->n_in == plan->n_in, "dense maps and plan disagree on sizes");
  FLY_REQUIRE(batch >= 0 && batch < (int64_t)INT32_MAX / 2, "batch out of range");
  if (batch) FLY_REQUIRE(x && ldx >= d->k && logits && wdl, "bad argument");
}

// The forward in blocks of at most `blk` boards, each using the scratch at ws (model_ws_block(blk) bytes).
void model_forward_blocks(const fly_plan &plan, const fly_dense &d, const void *x, bool x_f16, int64_t ldx,
                          int64_t batch, float input_gain, float *logits, float *wdl, void *ws, int64_t blk,
                          hipStream_t st) {
  char *base = static_cast<char *>(ws);
  float *u = reinterpret_cast<float *>(base);
  base += align256((size_t)plan.n_in * state_ld(blk, sizeof(float)) * sizeof(float));
  void *states = base;
  const size_t es = plan.mode == FLY_MODE_DEVIATION_F16 ? sizeof(_Float16) : sizeof(float);
  base += align256(2 * (size_t)plan.max_rows * (size_t)state_ld(blk, es) * es + 256);
  float *pieces = reinterpret_cast<float *>(base);   // the sums of split rows' pieces
  base += plan_pieces_bytes(plan, blk);
  void *scratch_ops = base;  // the encoder's operand split, then the head's
  const size_t xelem = x_f16 ? sizeof(_Float16) : sizeof(float);
  for (int64_t c0 = 0; c0 < batch; c0 += blk) {
    const int64_t nb = std::min(blk, batch - c0);
    const void *xb = static_cast<const char *>(x) + (size_t)c0 * ldx * xelem;
    float *lb = logits + c0 * d.n_moves, *wb = wdl + c0 * 3;
    const int64_t ldu = state_ld(nb, sizeof(float));
    const int64_t lds = state_ld(nb, es);
    // The encoder output stays float32 in both modes: only the deviation state is carried in float16.
    run_encoder(d, xb, x_f16, ldx, nb, input_gain, u, nullptr, ldu, scratch_ops, st);
    if (plan.mode == FLY_MODE_DEVIATION_F16) {
      const _Float16 *fin = run_cone_steps<_Float16, float>(plan, u, ldu, nb, true, states, pieces, st);
      run_head<_Float16>(d, fin, lds, plan.out_src.p, plan.cbase.p, nb, lb, wb, scratch_ops, st);
    } else {
      const float *fin = run_cone_steps<float, float>(plan, u, ldu, nb, true, states, pieces, st);
      run_head<float>(d, fin, lds, plan.out_src.p, plan.cbase.p, nb, lb, wb, scratch_ops, st);
    }
  }
}

}  // namespace
}  // namespace fly

// ---- the forward that allocates nothing -------------------------------------------------------------------------
// Its scratch is one file-scope device array per GPU (FLY_STATIC_SCRATCH_BYTES), held until the process ends.  In
// host code `scratch` names a host-side stand-in, never device memory: the array's address on the current device
// comes from hipGetSymbolAddress, once per device, and only that address is passed to kernels.
static __device__ __align__(256) char scratch[FLY_STATIC_SCRATCH_BYTES];

namespace fly {
namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices] = {};

// The scratch array's address on the current device (looked up on the first call on that device).
void *static_scratch() {
  const int dev = current_device();
  FLY_REQUIRE(dev >= 0 && dev < kMaxDevices, "device id out of range for the static scratch");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void *p = nullptr;
    FLY_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    FLY_REQUIRE(p != nullptr && aligned(p, 256), "the static scratch has no usable device address");
    g_scratch_ptr[dev] = p;
  }
  return g_scratch_ptr[dev];
}

// Boards per block that fit the static scratch: the whole batch if it fits, else the largest multiple of 64
// that does; 0 when not even min(batch, 64) boards fit.
int64_t static_block(const fly_plan &plan, const fly_dense &d, int64_t batch) {
  const size_t cap = FLY_STATIC_SCRATCH_BYTES;
  if (model_ws_block(plan, d, batch) <= cap) return batch;
  for (int64_t b = (batch - 1) / 64 * 64; b >= 64; b -= 64)
    if (model_ws_block(plan, d, b) <= cap) return b;
  return 0;
}

}  // namespace
}  // namespace fly

extern "C" int fly_model_forward_static(const fly_plan *plan, const fly_dense *d, const void *x, int32_t x_f16,
                                        int64_t ldx, int64_t batch, float input_gain, float *logits, float *wdl,
                                        void *stream) {
  return guard([&] {
    check_model_args(plan, d, x, ldx, batch, logits, wdl);
    if (!batch) return;
    const int64_t blk = static_block(*plan, *d, batch);
    FLY_REQUIRE(blk > 0, "fly_model_forward_static: one block of " + std::to_string(std::min<int64_t>(batch, 64)) +
                             " boards needs " + std::to_string(model_ws_block(*plan, *d, std::min<int64_t>(batch, 64))) +
                             " bytes of scratch, above the static array's " +
                             std::to_string((size_t)FLY_STATIC_SCRATCH_BYTES) + " (use fly_model_forward)");
    void *ws = static_scratch();
    NoLaunchEvents quiet;   // the profiler's launch events would be created here: this entry point creates nothing
    model_forward_blocks(*plan, *d, x, x_f16 != 0, ldx, batch, input_gain, logits, wdl, ws, blk, as_stream(stream));
  });
}

extern "C" size_t fly_model_workspace(const fly_plan *plan, const fly_dense *d, int64_t batch) {
  if (!plan || !d) return 0;
  // boards per block: the whole batch while the state stays below 2 GiB (io_block)
  return model_ws_block(*plan, *d, io_block(*plan, batch));
}

extern "C" int fly_model_forward(const fly_plan *plan, const fly_dense *d, const void *x, int32_t x_f16, int64_t ldx,
                                 int64_t batch, float input_gain, float *logits, float *wdl, void *ws, size_t ws_bytes,
                                 void *stream) {
  return guard([&] {
    check_model_args(plan, d, x, ldx, batch, logits, wdl);
    if (!batch) return;
    FLY_REQUIRE(ws && ws_bytes >= fly_model_workspace(plan, d, batch), "workspace too small");
    FLY_REQUIRE(aligned(ws, 256), "workspace must be 256-byte aligned");
    // Boards run in blocks whose state stays below 2 GiB (one block below about 6,400 boards in float16).
    model_forward_blocks(*plan, *d, x, x_f16 != 0, ldx, batch, input_gain, logits, wdl, ws, io_block(*plan, batch),
                         as_stream(stream));
  });
}
