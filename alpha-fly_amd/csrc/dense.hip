// Dense maps of the network on the matrix cores, and the whole-model forward.
//
//   encoder  u[m, b] = cast((sum_k W[m, k] x[b, k] + bias[m]) * gain)        chessfly/model.py:99-102
//   head     r[b, j] = clamp((c_base[j] + X_T[src_j, b] - mean_j) / sqrt(var_j + eps), -clip, clip)
//            logits[b, i] = (P r + bp)[i] + (F r + bf)[from_i] + (T r + bt)[to_i],  wdl = V r + bv
//                                                                            chessfly/model.py:51-58, 103-105
// The GEMM is C = A B^T with A row-major (the weight) and B produced by a loader functor, on 64x64
// output tiles of 4 waves (2x2 waves of 32x32, each 2x2 v_mfma_f32_16x16x4f32 tiles), K staged 16 at a
// time through LDS.  float32 matrix cores keep the dense maps float32-exact in their products.  The head's
// B loader reads the final recurrent state in place, so the output gather, the transpose to (B, n_out) and
// the normaliser never touch HBM as separate passes.
#include "common.hpp"

namespace fly {

int64_t state_ld(int64_t batch);
size_t io_workspace(const fly_plan &plan, int64_t batch);
template <typename S, typename U>
const S *run_cone_steps(const fly_plan &plan, const U *u, int64_t ldu, int64_t batch, void *ws, hipStream_t st);
void check_plan_device(const fly_plan *plan);

namespace {

typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int BM = 64, BN = 64, BK = 16, PAD = 4;
typedef float TileA[BK][BM + PAD];
typedef float TileB[BK][BN + PAD];

// A: row-major weight (M, ld), columns [0, K) used.
struct RowMajorA {
  const float *w;
  int64_t ld;
  __device__ __forceinline__ void tile(TileA &s, int64_t m0, int64_t k0, int64_t M, int64_t K, int tid) const {
    const int m = tid >> 2, kq = (tid & 3) * 4;
    const int64_t gm = m0 + m;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t k = k0 + kq + i;
      s[kq + i][m] = (gm < M && k < K) ? w[gm * ld + k] : 0.0f;
    }
  }
};

// B for the encoder: boards x (N, ld), B[n, k] = x[n, k].
struct BoardsB {
  const float *x;
  int64_t ld;
  __device__ __forceinline__ void tile(TileB &s, int64_t n0, int64_t k0, int64_t N, int64_t K, int tid) const {
    const int n = tid >> 2, kq = (tid & 3) * 4;
    const int64_t gn = n0 + n;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t k = k0 + kq + i;
      s[kq + i][n] = (gn < N && k < K) ? x[gn * ld + k] : 0.0f;
    }
  }
};

// B for the head: the normalised output activity r[n, k] read from the state (rows, lds) in place.
template <typename S>
struct NormalisedOutputsB {
  const S *state;        // null: no carried state
  int64_t lds;
  const int32_t *src;    // row of output k in the state (-1: none); null: row k
  const float *cbase;    // added to the state value; null: 0
  const float *mean, *var;
  float eps, clip;
  __device__ __forceinline__ void tile(TileB &s, int64_t n0, int64_t k0, int64_t N, int64_t K, int tid) const {
    const int k = tid >> 4, nq = (tid & 15) * 4;
    const int64_t gk = k0 + k;
    if (gk >= K) {
#pragma unroll
      for (int i = 0; i < 4; ++i) s[k][nq + i] = 0.0f;
      return;
    }
    const int32_t row = src ? src[gk] : (int32_t)gk;
    const float base = cbase ? cbase[gk] : 0.0f;
    const float mu = mean[gk];
    const float sd = sqrtf(var[gk] + eps);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t n = n0 + nq + i;
      float v = 0.0f;
      if (n < N) {
        const float r = base + ((state != nullptr && row >= 0) ? static_cast<float>(state[(int64_t)row * lds + n]) : 0.0f);
        v = fminf(fmaxf((r - mu) / sd, -clip), clip);
      }
      s[k][nq + i] = v;
    }
  }
};

template <typename S>
struct EncoderEpilogue {
  const float *bias;
  float gain;
  S *u;
  int64_t ldu;
  __device__ __forceinline__ void operator()(int64_t m, int64_t n, float v) const {
    u[m * ldu + n] = static_cast<S>((v + bias[m]) * gain);
  }
};

// C^T rows: ct[n, moff + m] = C[m, n] (one row of all head outputs per board).
struct HeadEpilogue {
  float *ct;
  int64_t ldc, moff;
  __device__ __forceinline__ void operator()(int64_t m, int64_t n, float v) const { ct[n * ldc + moff + m] = v; }
};

template <class AL, class BL, class EP>
__global__ __launch_bounds__(256) void k_gemm(int64_t M, int64_t N, int64_t K, const AL A, const BL B, const EP ep) {
  __shared__ TileA As;
  __shared__ TileB Bs;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * BN;
  v4f acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};
  for (int64_t k0 = 0; k0 < K; k0 += BK) {
    A.tile(As, m0, k0, M, K, tid);
    B.tile(Bs, n0, k0, N, K, tid);
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < BK; kk += 4) {
      const int kr = kk + (lane >> 4);
      float a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) a[i] = As[kr][wm * 32 + i * 16 + (lane & 15)];
#pragma unroll
      for (int j = 0; j < 2; ++j) b[j] = Bs[kr][wn * 32 + j * 16 + (lane & 15)];
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t m = m0 + wm * 32 + i * 16 + 4 * (lane >> 4) + r;
        const int64_t n = n0 + wn * 32 + j * 16 + (lane & 15);
        if (m < M && n < N) ep(m, n, acc[i][j][r]);
      }
}

template <class AL, class BL, class EP>
void gemm(int64_t M, int64_t N, int64_t K, const AL &A, const BL &B, const EP &ep, hipStream_t st) {
  if (M == 0 || N == 0) return;
  const int64_t gy = (M + BM - 1) / BM, gx = (N + BN - 1) / BN;
  FLY_REQUIRE(gy < 65536 && gx < INT32_MAX, "GEMM grid too large");
  hipLaunchKernelGGL((k_gemm<AL, BL, EP>), dim3((unsigned)gx, (unsigned)gy), dim3(256), 0, st, M, N, K, A, B, ep);
  check_launch("gemm");
}

// logits[n, i] = (ct[n, i] + bp[i]) + (ct[n, M + f] + bf[f]) + (ct[n, M + 64 + t] + bt[t]); wdl from the last 3.
__global__ void k_assemble(const float *__restrict__ ct, int64_t ldc, int64_t n_moves, const float *__restrict__ bp,
                           const float *__restrict__ bf, const float *__restrict__ bt, const float *__restrict__ bv,
                           const int32_t *__restrict__ mfrom, const int32_t *__restrict__ mto, int64_t batch,
                           float *__restrict__ logits, float *__restrict__ wdl) {
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  for (int64_t n = blockIdx.y; n < batch; n += gridDim.y) {
    const float *row = ct + n * ldc;
    if (i < n_moves) {
      const int32_t f = min(max(mfrom[i], 0), 63), t = min(max(mto[i], 0), 63);  // squares are 0..63
      logits[n * n_moves + i] = ((row[i] + bp[i]) + (row[n_moves + f] + bf[f])) + (row[n_moves + 64 + t] + bt[t]);
    }
    if (i < 3) wdl[n * 3 + i] = row[n_moves + 128 + i] + bv[i];
  }
}

int64_t head_ld(const fly_head_desc &h) { return round_up(h.n_moves + 131, 4); }

size_t head_ws(const fly_head_desc &h, int64_t batch) { return (size_t)batch * head_ld(h) * sizeof(float) + 256; }

void check_head(const fly_head_desc *h) {
  FLY_REQUIRE(h != nullptr, "head is null");
  FLY_REQUIRE(h->n_out > 0 && h->n_moves > 0, "empty head");
  FLY_REQUIRE(h->norm_mean && h->norm_var && h->policy_w && h->policy_b && h->from_w && h->from_b && h->to_w &&
                  h->to_b && h->value_w && h->value_b && h->move_from && h->move_to,
              "head has a null pointer");
}

template <typename S>
void run_head(const fly_head_desc &h, const NormalisedOutputsB<S> &B, int64_t batch, float *ct, float *logits,
              float *wdl, hipStream_t st) {
  const int64_t ldc = head_ld(h), K = h.n_out;
  LaunchTimer timer(FLY_K_HEAD, st);
  gemm(h.n_moves, batch, K, RowMajorA{h.policy_w, K}, B, HeadEpilogue{ct, ldc, 0}, st);
  gemm(64, batch, K, RowMajorA{h.from_w, K}, B, HeadEpilogue{ct, ldc, h.n_moves}, st);
  gemm(64, batch, K, RowMajorA{h.to_w, K}, B, HeadEpilogue{ct, ldc, h.n_moves + 64}, st);
  gemm(3, batch, K, RowMajorA{h.value_w, K}, B, HeadEpilogue{ct, ldc, h.n_moves + 128}, st);
  const dim3 grid(blocks_for(h.n_moves, 256), (unsigned)std::min<int64_t>(batch, 65535));
  hipLaunchKernelGGL(k_assemble, grid, dim3(256), 0, st, ct, ldc, h.n_moves, h.policy_b, h.from_b, h.to_b, h.value_b,
                     h.move_from, h.move_to, batch, logits, wdl);
  check_launch("head assembly");
}

template <typename S>
void run_encoder(const float *x, int64_t ldx, int64_t batch, int64_t k, const float *w, int64_t ldw, const float *b,
                 int64_t n_in, float gain, S *u, int64_t ldu, hipStream_t st) {
  LaunchTimer timer(FLY_K_ENCODER, st);
  gemm(n_in, batch, k, RowMajorA{w, ldw}, BoardsB{x, ldx}, EncoderEpilogue<S>{b, gain, u, ldu}, st);
}

size_t align256(size_t x) { return (x + 255) / 256 * 256; }

}  // namespace
}  // namespace fly

using namespace fly;

extern "C" int fly_encoder(const float *x, int64_t ldx, int64_t batch, int64_t k, const float *w, int64_t ldw,
                           const float *b, int64_t n_in, float gain, void *u, int64_t ldu, int32_t out_f16,
                           void *stream) {
  return guard([&] {
    FLY_REQUIRE(batch >= 0 && n_in >= 0 && k >= 0, "negative size");
    if (!batch || !n_in) return;
    FLY_REQUIRE(x && w && b && u, "null argument");
    FLY_REQUIRE(ldx >= k && ldw >= k && ldu >= batch, "leading dimension too small");
    if (out_f16)
      run_encoder<_Float16>(x, ldx, batch, k, w, ldw, b, n_in, gain, static_cast<_Float16 *>(u), ldu, as_stream(stream));
    else
      run_encoder<float>(x, ldx, batch, k, w, ldw, b, n_in, gain, static_cast<float *>(u), ldu, as_stream(stream));
  });
}

extern "C" size_t fly_head_workspace(const fly_head_desc *head, int64_t batch) {
  return head ? head_ws(*head, batch) : 0;
}

extern "C" int fly_head(const fly_head_desc *head, const float *r, int64_t ldr, int64_t batch, float *logits,
                        float *wdl, void *ws, size_t ws_bytes, void *stream) {
  return guard([&] {
    check_head(head);
    FLY_REQUIRE(batch >= 0, "negative batch");
    if (!batch) return;
    FLY_REQUIRE(r && ldr >= batch && logits && wdl, "bad argument");
    FLY_REQUIRE(ws && ws_bytes >= head_ws(*head, batch), "workspace too small");
    NormalisedOutputsB<float> B{r, ldr, nullptr, nullptr, head->norm_mean, head->norm_var, head->norm_eps, head->norm_clip};
    run_head<float>(*head, B, batch, static_cast<float *>(ws), logits, wdl, as_stream(stream));
  });
}

extern "C" size_t fly_model_workspace(const fly_plan *plan, const fly_head_desc *head, int64_t batch) {
  if (!plan || !head) return 0;
  return align256((size_t)plan->n_in * state_ld(batch) * sizeof(float)) + align256(io_workspace(*plan, batch)) +
         align256(head_ws(*head, batch));
}

extern "C" int fly_model_forward(const fly_plan *plan, const fly_head_desc *head, const float *x, int64_t ldx,
                                 int64_t batch, int64_t k, const float *enc_w, int64_t ldw, const float *enc_b,
                                 float input_gain, float *logits, float *wdl, void *ws, size_t ws_bytes, void *stream) {
  return guard([&] {
    check_plan_device(plan);
    check_head(head);
    FLY_REQUIRE(!plan->full, "the model forward needs a light-cone plan");
    FLY_REQUIRE(head->n_out == plan->n_out, "head and plan disagree on the number of outputs");
    FLY_REQUIRE(batch >= 0 && batch < (int64_t)INT32_MAX / 2, "batch out of range");
    if (!batch) return;
    FLY_REQUIRE(x && ldx >= k && logits && wdl, "bad argument");
    FLY_REQUIRE(plan->n_in == 0 || (enc_w && enc_b && ldw >= k), "bad encoder");
    FLY_REQUIRE(ws && ws_bytes >= fly_model_workspace(plan, head, batch), "workspace too small");
    FLY_REQUIRE(aligned(ws, 256), "workspace must be 256-byte aligned");
    hipStream_t st = as_stream(stream);
    const int64_t ldu = state_ld(batch);
    const bool dev = plan->mode == FLY_MODE_DEVIATION_F16;
    char *base = static_cast<char *>(ws);
    void *u = base;
    base += align256((size_t)plan->n_in * ldu * sizeof(float));
    void *states = base;
    base += align256(io_workspace(*plan, batch));
    float *ct = reinterpret_cast<float *>(base);
    const int64_t lds = state_ld(batch);
    // The encoder output stays float32 in both modes: only the deviation state is carried in float16.
    run_encoder<float>(x, ldx, batch, k, enc_w, ldw, enc_b, plan->n_in, input_gain, static_cast<float *>(u), ldu, st);
    if (dev) {
      const _Float16 *fin = run_cone_steps<_Float16, float>(*plan, static_cast<float *>(u), ldu, batch, states, st);
      NormalisedOutputsB<_Float16> B{fin, lds, plan->out_src.p, plan->cbase.p, head->norm_mean, head->norm_var,
                                     head->norm_eps, head->norm_clip};
      run_head<_Float16>(*head, B, batch, ct, logits, wdl, st);
    } else {
      const float *fin = run_cone_steps<float, float>(*plan, static_cast<float *>(u), ldu, batch, states, st);
      NormalisedOutputsB<float> B{fin, lds, plan->out_src.p, plan->cbase.p, head->norm_mean, head->norm_var,
                                  head->norm_eps, head->norm_clip};
      run_head<float>(*head, B, batch, ct, logits, wdl, st);
    }
  });
}
