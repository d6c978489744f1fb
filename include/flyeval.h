/*
 * flyeval.h - C ABI of the MI355X (gfx950) forward evaluator of the connectome chess network.
 *
 * Every entry point returns an int status (FLY_OK = 0) and never throws; on failure
 * fly_last_error() returns a message for the calling thread.  Pointers named *_dev are device
 * pointers owned by the caller (torch tensors on the Python side); the library never frees them.
 * The library owns only what its create functions return (cones and plans) and frees it in the
 * matching destroy.  `stream` is a hipStream_t passed as void* (torch's current stream); every
 * launch goes on it.  Only the create functions synchronise (they read sizes back to the host);
 * the forward entry points are asynchronous.  Index arrays are int32, the graph is CSR of
 * W[post, pre] (row = postsynaptic neuron).  A created object is immutable apart from the cone's cache of sweep
 * tables, which takes a lock: plans may be created and forwards run from several threads, each with its own
 * workspace and stream.  fly_set_tuning changes the defaults of objects created afterwards.
 *
 * Reference interfaces replaced (paths relative to the alpha-fly repository):
 *   fly_cone_*            chessfly/brain.py:126-173 LightCone, :102-123 _SubMatrix, :232-236 light_cone
 *   fly_edge_weights      chessfly/brain.py:201-202 ConnectomeRNN.edge_weights
 *   fly_plan_create       chessfly/brain.py:257-270 (_forward_io_half cache) and :295-306 (float32 cache),
 *                         :238-252 _constants
 *   fly_plan_create_full  chessfly/brain.py:215-216 (per-call weights of the literal recurrence)
 *   fly_forward_io        chessfly/brain.py:282-329 ConnectomeRNN.forward_io (and :254-280); _f64 in float64
 *   fly_forward_literal   chessfly/brain.py:211-223 ConnectomeRNN.forward (no-grad branch); _f64 and _f16 in those
 *                         dtypes
 *   fly_plan_step         chessfly/brain.py:273-277 and :310-313 (one step of forward_io; :219-220 one literal step)
 *   fly_dense_create      chessfly/model.py:79-93 (the encoder and head weights, as the matrix cores read them)
 *   fly_encoder           chessfly/model.py:99-102 (encoder linear map, input gain, cast, transpose)
 *   fly_head              chessfly/model.py:103-105 and :51-58 (RunningNorm eval, policy/from/to/value)
 *   fly_model_forward     chessfly/model.py:95-105 FlyChessNet.forward (no-grad, device inputs)
 *   fly_evaluator_outputs chessfly/model.py:120-128 and :107-110 (Evaluator.submit's half cast or legal gather,
 *                         expected_value)
 *   fly_evaluator_download chessfly/model.py:130-131 (Evaluator.result's copies of the answers to the host)
 *   fly_spmm, fly_sddmm   chessfly/brain.py:66-99 (_SparseRecurrent forward, grad_h and grad_w); fly_spmm_swept the
 *                         forward product as a banded sweep; _f64 in float64
 *   fly_sweep_*, fly_plan_sweep_info  no counterpart (cuSPARSE keeps its own analysis of a structure): the banded
 *                         sweep's tables of one CSR structure
 *   fly_transposed_backward  chessfly/brain.py:79-99 (_SparseRecurrent.backward: grad_h and grad_w in one pass;
 *                         _swept as a banded sweep)
 *   fly_spmv_work         chessfly/brain.py:79-99 and :238-252 (grad_h = A^T grad_y of the resting trajectory's
 *                         one-column products, under autograd)
 *   fly_rest_*            chessfly/brain.py:238-252 (_constants under autograd: the resting trajectory and the
 *                         constant drives k_t, forward and backward)
 *   fly_gather_values     chessfly/brain.py:123, 208, 248, 293 (w[op.edges], w[t_order]: a sub-matrix's values)
 *   fly_gather_records    the same, beside the structure's columns (the swept products' records)
 *   fly_train_step_*      chessfly/brain.py:313-327 under autograd (clamp, index_add, index_copy, lerp and their
 *                         gradients)
 *   fly_model_forward_static  no counterpart: the model forward for callers that cannot allocate
 *   fly_profile_*, fly_set_tuning, fly_get_tuning  measurement and launch-shape choices (timing scripts)
 */
#ifndef FLYEVAL_H
#define FLYEVAL_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FLY_ABI_VERSION 2

enum fly_status {
    FLY_OK = 0,
    FLY_ERR_INVALID = 1,   /* bad argument: null pointer, size, alignment, index out of range */
    FLY_ERR_HIP = 2,       /* a HIP runtime call failed */
    FLY_ERR_INTERNAL = 3
};

/* State arithmetic of a plan. */
enum fly_mode {
    FLY_MODE_DEVIATION_F16 = 0,  /* fp16 deviation from the float32 resting trajectory (brain.py:254-280) */
    FLY_MODE_F32 = 1             /* float32 light-cone state (brain.py:295-329) */
};

typedef struct fly_cone fly_cone;
typedef struct fly_plan fly_plan;
typedef struct fly_sweep fly_sweep;

int fly_abi_version(void);
const char *fly_last_error(void);

/* ---- light cone (integer, bit-exact with chessfly/brain.py:126-173) ------------------------------
 * crow_dev (n+1), pre_dev (n_edges): CSR of W; in_idx_dev (n_in), out_idx_dev (n_out): neuron ids.
 * flags: 0 prunes to the light cone; FLY_CONE_UNPRUNED computes every neuron at every step t >= 1 (the
 * same function without pruning).  Validates every index on the device first (FLY_ERR_INVALID if any is
 * out of range). */
#define FLY_CONE_UNPRUNED 1
int fly_cone_create(int64_t n, int64_t n_edges, const int32_t *crow_dev, const int32_t *pre_dev,
                    const int32_t *in_idx_dev, int64_t n_in, const int32_t *out_idx_dev, int64_t n_out,
                    int32_t steps, int32_t flags, void *stream, fly_cone **out);
int fly_cone_destroy(fly_cone *cone);
/* rows[t] = |R_t| for t = 0..steps; nnz[t] = non-zeros of A_t (0 where A_t is None); has_op[t] = 1 where
 * A_t exists (R_{t-1} non-empty).  Arrays have steps+1 entries; any may be NULL. */
int fly_cone_sizes(const fly_cone *cone, int64_t *rows, int64_t *nnz, int32_t *has_op);
/* R_t, sorted neuron ids (|R_t| entries). */
int fly_cone_rows(const fly_cone *cone, int32_t t, int32_t *rows_dev, void *stream);
/* Step t >= 1: crow (|R_t|+1), local column (nnz_t), global edge id (nnz_t) of A_t (NULL skips an array;
 * all three are skipped when A_t is None), prev (|R_t|: position in R_{t-1}, -1 if not carried) and usrc
 * (|R_t|: position in in_idx, -1 if the row is not an input). */
int fly_cone_step(const fly_cone *cone, int32_t t, int32_t *crow_dev, int32_t *col_dev, int32_t *edge_dev,
                  int32_t *prev_dev, int32_t *usrc_dev, void *stream);
/* out_src (n_out): position of out_idx[j] in R_T, -1 if absent. */
int fly_cone_outputs(const fly_cone *cone, int32_t *out_src_dev, void *stream);

/* ---- weights ----------------------------------------------------------------------------------- */
/* w = sign * w0 * exp(log_gain), n_edges entries. */
int fly_edge_weights(const float *sign_dev, const float *w0_dev, const float *log_gain_dev, int64_t n_edges,
                     float *w_dev, void *stream);

/* Weight-set plan for forward_io: per-step sub-matrices with float32 values, per-row constants and the
 * resting trajectory, from the cone and the graph (crow/pre as given to fly_cone_create), edge weights w
 * (n_edges), bias and alpha_logit (n).  The plan keeps no pointer to its inputs: they may be freed afterwards.
 * Activity is clamped to [0, h_max]; h_max = +INFINITY clamps only below (the reference's h_max=None,
 * chessfly/brain.py:178-182, 221).  A negative or NaN h_max is FLY_ERR_INVALID.
 * The plan captures the tuning (fly_set_tuning) current at its creation.  Long-row steps run as a banded sweep
 * over tables that depend only on the cone's structure: the cone builds them on the first plan that needs them
 * and every later plan of the cone (each new weight version) shares them, so only that first plan pays for them.
 * A plan holds a reference to them, so it outlives fly_cone_destroy. */
int fly_plan_create(const fly_cone *cone, const int32_t *crow_dev, const int32_t *pre_dev, const float *w_dev,
                    const float *bias_dev, const float *alpha_logit_dev, float h_max, int32_t mode,
                    void *stream, fly_plan **out);
/* Plan for the literal recurrence over the whole matrix (mode FLY_MODE_F32, every row carried).  sweep: the banded-
 * sweep tables of the matrix's structure (fly_sweep_create over crow/pre), shared by every plan of
 * the structure; NULL runs every step on the grouped kernel. */
int fly_plan_create_full(int64_t n, int64_t n_edges, const int32_t *crow_dev, const int32_t *pre_dev,
                         const float *w_dev, const float *alpha_logit_dev, float h_max, const fly_sweep *sweep,
                         void *stream, fly_plan **out);
int fly_plan_destroy(fly_plan *plan);
/* c_T[out_idx] (n_out floats): the outputs of a network that sees no position. */
int fly_plan_resting(const fly_plan *plan, float *c_out_dev, void *stream);
/* How step t runs (t = 1 for a literal plan): info[7] = {positions of the sweep order, pieces of split rows, rows
 * split, rows per wave, bands, workgroups, an identity of the tables (equal for plans that share them)}, all 0 when
 * the step does not sweep. */
int fly_plan_sweep_info(const fly_plan *plan, int32_t t, int64_t *info);
/* The plan's sub-matrix A_t as the step kernels read it, the cached per-step matrix of chessfly/brain.py:267-268
 * (fp16 path) and :303 (float32 path): row pointer (|R_t|+1), local column and float32 value (nnz_t each), in
 * W's edge order.  Nothing is written where A_t does not exist; NULL skips an array.  A literal plan has one
 * matrix, t = 1 (W itself). */
int fly_plan_matrix(const fly_plan *plan, int32_t t, int32_t *rowptr_dev, int32_t *col_dev, float *val_dev,
                    void *stream);

/* ---- banded-sweep tables of one structure ----------------------------------------------------- */
/* No counterpart in the reference (cuSPARSE keeps its own analysis).  The tables a swept product or literal step
 * reads for a CSR structure: rowptr (nrows+1) and col (nnz) over ncols columns (rows of the operand).  Rows longer
 * than 3 x the mean + 10 non-zeros are split into pieces of at most that many, each a share of every band;
 * the step adds a split row's pieces in piece order.  Captures the tuning current at creation (sweep_paired > 0:
 * the order is searched for waves that walk two rows per pass).  *out = NULL (FLY_OK) when the structure is too small to
 * sweep (by size: over 32,768 columns, at least 65,536 rows and 32 non-zeros per row).  Synchronises.
 * fly_sweep_info: info[7] as fly_plan_sweep_info's. */
int fly_sweep_create(const int32_t *rowptr_dev, const int32_t *col_dev, int64_t nrows, int64_t nnz, int64_t ncols,
                     void *stream, fly_sweep **out);
int fly_sweep_destroy(fly_sweep *sweep);
int fly_sweep_info(const fly_sweep *sweep, int64_t *info);

/* ---- forward ----------------------------------------------------------------------------------- */
/* Bytes of scratch the forward entry points need for `batch` columns (pass at least this many).  A batch whose
 * state would pass 2 GiB runs internally as column blocks below it, and the workspace is sized for one block. */
size_t fly_forward_io_workspace(const fly_plan *plan, int64_t batch);
/* u_in (n_in, ldu): __half for FLY_MODE_DEVIATION_F16, float for FLY_MODE_F32.
 * out (n_out, ldo) float32 = forward_io(u_in)[out rows]. */
int fly_forward_io(const fly_plan *plan, const void *u_in_dev, int64_t ldu, int64_t batch, float *out_dev,
                   int64_t ldo, void *workspace_dev, size_t workspace_bytes, void *stream);
/* forward_io with u_in float64 (chessfly/brain.py:295-329 in u_in's dtype): a FLY_MODE_F32 plan's float32 cache
 * (k_t, c_t, alphas, A_t values) widens exactly, as the reference's .to(dtype) of its float32 cache does, and the
 * state, sums, clamp and lerp are float64.  u_in (n_in, ldu) and out (n_out, ldo) float64. */
size_t fly_forward_io_f64_workspace(const fly_plan *plan, int64_t batch);
int fly_forward_io_f64(const fly_plan *plan, const double *u_in_dev, int64_t ldu, int64_t batch, double *out_dev,
                       int64_t ldo, void *workspace_dev, size_t workspace_bytes, void *stream);
/* Literal recurrence (plan from fly_plan_create_full): u (n, ldu) float32 is updated in place to u + bias
 * (as the reference's no-grad path does), then h_steps (n, ldh) = steps updates from h = 0. */
size_t fly_forward_literal_workspace(const fly_plan *plan, int64_t batch);
int fly_forward_literal(const fly_plan *plan, float *u_dev, int64_t ldu, const float *bias_dev, int64_t batch,
                        int32_t steps, float *h_dev, int64_t ldh, void *workspace_dev, size_t workspace_bytes,
                        void *stream);
/* The same recurrence in float64 (chessfly/brain.py:215-223 with u float64: the float32 weights, alphas and bias
 * widen exactly, and every sum, clamp and lerp is float64; the reference's tests run it this way).  u (n, ldu) is
 * updated in place to u + bias; h (n, ldh) float64. */
size_t fly_forward_literal_f64_workspace(const fly_plan *plan, int64_t batch);
int fly_forward_literal_f64(const fly_plan *plan, double *u_dev, int64_t ldu, const float *bias_dev, int64_t batch,
                            int32_t steps, double *h_dev, int64_t ldh, void *workspace_dev, size_t workspace_bytes,
                            void *stream);
/* The same recurrence in float16 (chessfly/brain.py:213-223 with u float16): u and h are __half, u += bias rounded to
 * float16 in place, the state is float16 with float32 sums.  The reference rounds the weights to u's dtype: pass a
 * plan built from float16-rounded weights for that. */
size_t fly_forward_literal_f16_workspace(const fly_plan *plan, int64_t batch);
int fly_forward_literal_f16(const fly_plan *plan, void *u_dev, int64_t ldu, const float *bias_dev, int64_t batch,
                            int32_t steps, void *h_dev, int64_t ldh, void *workspace_dev, size_t workspace_bytes,
                            void *stream);

/* One state step of a plan, the per-step op of chessfly/brain.py:273-277 (float16 deviation: s = A_t d_{t-1},
 * index_add_ of the input, FUSED_DEVIATION) and :310-313 (float32: A_t h + input, FUSED_UPDATE with k_t):
 * xout (|R_t|, ldo) from xprev (|R_{t-1}|, ldx) and the input drive u_in (n_in, ldu).  States and u_in are __half
 * (the deviation from the resting trajectory) for FLY_MODE_DEVIATION_F16 and float for FLY_MODE_F32.  xprev is
 * NULL when R_{t-1} is empty (t = 1) and required otherwise; u_in NULL adds no input.  For a plan from
 * fly_plan_create_full, t is 1 and the step is one literal update of every row, x = clamp(W h + u, 0, h_max),
 * h' = lerp(h, x, alpha), with u_in (n, ldu) holding u + bias and xprev NULL for h = 0.  Only columns
 * [0, batch) of the caller's rows are read or written.  workspace: fly_plan_step_workspace bytes, 256-byte aligned
 * (the sums of a swept step's split rows; 0 bytes and NULL for other steps). */
size_t fly_plan_step_workspace(const fly_plan *plan, int32_t t, int64_t batch);
int fly_plan_step(const fly_plan *plan, int32_t t, const void *xprev_dev, int64_t ldx, const void *u_in_dev,
                  int64_t ldu, int64_t batch, void *xout_dev, int64_t ldo, void *workspace_dev,
                  size_t workspace_bytes, void *stream);

/* ---- dense maps -------------------------------------------------------------------------------- */
/* Weights of the read-out: RunningNorm statistics and the four linear maps over the n_out outputs. */
typedef struct fly_head_desc {
    int64_t n_out;              /* 2,333 */
    int64_t n_moves;            /* 4,168 */
    const float *norm_mean;     /* (n_out) */
    const float *norm_var;      /* (n_out) */
    float norm_eps;
    float norm_clip;
    const float *policy_w;      /* (n_moves, n_out) row-major */
    const float *policy_b;      /* (n_moves) */
    const float *from_w;        /* (64, n_out) */
    const float *from_b;
    const float *to_w;          /* (64, n_out) */
    const float *to_b;
    const float *value_w;       /* (3, n_out) */
    const float *value_b;
    const int32_t *move_from;   /* (n_moves) squares 0..63 */
    const int32_t *move_to;
} fly_head_desc;

typedef struct fly_dense fly_dense;

/* Dense plan: the encoder (n_in, ldw) over its first k feature columns, its bias, and the head, copied and
 * split into fp16 hi/lo pairs for the matrix cores (rebuild it when any of these weights changes).
 * Validates the move squares (FLY_ERR_INVALID outside 0..63). */
int fly_dense_create(const fly_head_desc *head, const float *enc_w_dev, int64_t ldw, int64_t k,
                     const float *enc_b_dev, int64_t n_in, void *stream, fly_dense **out);
int fly_dense_destroy(fly_dense *dense);

/* u (n_in, ldu) = cast((x[:, :k] W[:, :k]^T + b) * gain): x (batch, ldx) float32, or __half when x_f16 != 0
 * (the search's boards, model.py:124, widened exactly as .float() does); out_f16 != 0 stores __half, else float. */
size_t fly_encoder_workspace(const fly_dense *dense, int64_t batch);
int fly_encoder(const fly_dense *dense, const void *x_dev, int32_t x_f16, int64_t ldx, int64_t batch, float gain,
                void *u_dev, int64_t ldu, int32_t out_f16, void *workspace_dev, size_t workspace_bytes, void *stream);

/* logits (batch, n_moves) and wdl (batch, 3), float32 row-major, from the output activity
 * r (n_out, ldr) float32 (column b = board b), through the eval-mode normaliser. */
size_t fly_head_workspace(const fly_dense *dense, int64_t batch);
int fly_head(const fly_dense *dense, const float *r_dev, int64_t ldr, int64_t batch, float *logits_dev,
             float *wdl_dev, void *workspace_dev, size_t workspace_bytes, void *stream);

/* FlyChessNet.forward: x (batch, ldx) float32 (or __half, x_f16 != 0) -> logits (batch, n_moves), wdl (batch, 3).
 * The plan's mode selects the state arithmetic; the encoder output (times input_gain) is kept in float32 in
 * both modes. */
size_t fly_model_workspace(const fly_plan *plan, const fly_dense *dense, int64_t batch);
int fly_model_forward(const fly_plan *plan, const fly_dense *dense, const void *x_dev, int32_t x_f16, int64_t ldx,
                      int64_t batch, float input_gain, float *logits_dev, float *wdl_dev, void *workspace_dev,
                      size_t workspace_bytes, void *stream);

/* No counterpart in the reference.  For callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc): fly_model_forward with the same inputs, outputs and
 * results, whose scratch is a static device array of FLY_STATIC_SCRATCH_BYTES that the library holds on each GPU it
 * runs on until the process ends; the call allocates nothing.  Boards run in blocks sized to that array: the full-scale
 * network (166,700 neurons) in blocks of 256 boards for FLY_MODE_DEVIATION_F16 and 128 for FLY_MODE_F32.
 * FLY_ERR_INVALID when not even a block of min(batch, 64) boards fits.  Every call on one GPU shares that GPU's array
 * and nothing in it must start at zero; calls that overlap on one GPU (other streams or threads) race, so the caller
 * serialises them.  Launches under it record no profiler events. */
#define FLY_STATIC_SCRATCH_BYTES ((size_t)256 << 20)
int fly_model_forward_static(const fly_plan *plan, const fly_dense *dense, const void *x_dev, int32_t x_f16,
                             int64_t ldx, int64_t batch, float input_gain, float *logits_dev, float *wdl_dev,
                             void *stream);

/* What the search's evaluate callable returns (chessfly/model.py:120-128), from logits (batch, n_moves) and
 * wdl (batch, 3), float32 row-major:
 *   values[b] = P(win) - P(loss) under the softmax of wdl[b] (expected_value, model.py:107-110);
 *   rows == NULL (lazy search): logits16 (batch, n_moves) __half = logits rounded to nearest even;
 *   else (eager search): legal[m] = logits[rows[m], cols[m]] for m < n_legal, rows/cols int64 indexed as
 *   torch does (negative values count from the end).
 * An index outside the shape cannot be reported before the kernel has run, so the kernel writes NaN for
 * that entry and sets *bad_dev to 1; *bad_dev is 0 otherwise (the call clears it first).  The caller reads
 * it back with the outputs. */
int fly_evaluator_outputs(const float *logits_dev, const float *wdl_dev, int64_t batch, int64_t n_moves,
                          const int64_t *rows_dev, const int64_t *cols_dev, int64_t n_legal, void *logits16_dev,
                          float *legal_dev, float *values_dev, int32_t *bad_dev, void *stream);
/* The answers' trip to the host (chessfly/model.py:130-131, Evaluator.result's .cpu() of the policy and values):
 * bytes from device memory to pinned host memory (hipHostMalloc, torch pin_memory=True), both 16-byte aligned,
 * as a kernel on `stream` whose `workgroups` (0: the default, 16) write through the host buffer's device address.
 * Any other kind of source or destination is FLY_ERR_INVALID.
 * Stores to host memory wait on the bus and hold up the other work of the CUs that issue them; a copy queued on
 * a stream of its own while the next batch computes therefore keeps to a few CUs. */
int fly_evaluator_download(const void *src_dev, void *dst_host, size_t bytes, int32_t workgroups, void *stream);

/* ---- training: the sparse products of the differentiable recurrence ----------------------------- */
/* chessfly/brain.py:66-99 (_SparseRecurrent), float32.  A is CSR (rowptr nrows+1, col/val nnz, int32 and
 * float); operands are row-major with the batch fastest.
 *   fly_spmm:  y (nrows, ldy) = A x (accumulate != 0: y += A x), x (ncols, ldx).  The values are val[e], or
 *              val[val_ids[e]] when val_ids is given (a sub-matrix read from the whole weight vector of n_val
 *              entries; an index past it reads 0).  The
 *              forward product, and with the transposed structure of A the state gradient A^T grad_y.
 *   fly_sddmm: out[e] = sum_b g[row_e, b] x[col_e, b] for every non-zero e, CSR order: the per-synapse
 *              gradient of y = A x with g = dL/dy.  With ids (distinct), out[ids[e]] instead (a sub-matrix's
 *              gradient straight into the whole weight vector); accumulate != 0 adds; out holds n_out entries and slots at
 *              or past it are skipped.  out must not overlap g.
 *   fly_spmm_swept: the forward product as a banded sweep of x's rows (the state step's swept kernel, storing
 *              each row's sums) over the tables of fly_sweep_create: y = A x from the
 *              structure's nnz {column, weight bits} records (int2, CSR order), for batches that are multiples of
 *              4 with 16-byte aligned rows; workspace: fly_spmm_swept_workspace bytes, 256-byte aligned (the sums
 *              of split rows' pieces; 0 without).  nnz must be the structure's.
 * Gathered operands must be below 2 GiB; rows and columns below 2^24; column indices are not range-checked
 * (a wrong index reads wrong data, never outside x). */
size_t fly_spmm_swept_workspace(const fly_sweep *sweep, int64_t batch);
int fly_spmm_swept(const fly_sweep *sweep, const void *records_dev, int64_t nnz, const float *x_dev, int64_t ldx,
                   int64_t batch, float *y_dev, int64_t ldy, void *workspace_dev, size_t workspace_bytes,
                   void *stream);
int fly_spmm(const int32_t *rowptr_dev, const int32_t *col_dev, const float *val_dev, const int32_t *val_ids_dev,
             int64_t n_val, int64_t nrows, int64_t ncols, const float *x_dev, int64_t ldx, int64_t batch,
             float *y_dev, int64_t ldy, int32_t accumulate, void *stream);
int fly_sddmm(const int32_t *rowptr_dev, const int32_t *col_dev, int64_t nrows, int64_t ncols, const float *g_dev,
              int64_t ldg, const float *x_dev, int64_t ldx, int64_t batch, float *out_dev, int64_t n_out,
              const int32_t *ids_dev, int32_t accumulate, void *stream);

/* The same products in float64, for networks converted to float64 (the reference's .double() test modules,
 * tests/test_core.py:28-44 and :309-338, which run ConnectomeRNN under autograd in float64): y (nrows, ldy) (+)= A x with
 * A's values val[e] or val[val_ids[e]], and out[ids ? ids[e] : e] (+)= sum_b g[row_e, b] x[col_e, b].  nnz bounds
 * the row pointer; values past n_val, columns past ncols and ids past n_out are skipped.  Each sum runs in CSR
 * order. */
int fly_spmm_f64(const int32_t *rowptr_dev, const int32_t *col_dev, int64_t nnz, const double *val_dev,
                 const int32_t *val_ids_dev, int64_t n_val, int64_t nrows, int64_t ncols, const double *x_dev,
                 int64_t ldx, int64_t batch, double *y_dev, int64_t ldy, int32_t accumulate, void *stream);
int fly_sddmm_f64(const int32_t *rowptr_dev, const int32_t *col_dev, int64_t nnz, int64_t nrows, int64_t ncols,
                  const double *g_dev, int64_t ldg, const double *x_dev, int64_t ldx, int64_t batch, double *out_dev,
                  int64_t n_out, const int32_t *ids_dev, int32_t accumulate, void *stream);

/* out[i] = w[ids[i]] for i < n (a sub-matrix's values in its own or its transpose's order); ids at or past n_w
 * read 0.  n_w below 2^29. */
int fly_gather_values(const float *w_dev, int64_t n_w, const int32_t *ids_dev, int64_t n, float *out_dev,
                      void *stream);
/* The same gather into a structure's {column, value bits} records, as fly_spmm_swept and
 * fly_transposed_backward_swept read them: records[i] = {col[i], w[ids[i]]} (w[i] with ids NULL; ids at or past n_w
 * give 0), records 8-byte aligned (chessfly/brain.py:123, 208: w[op.edges] beside the structure's columns). */
int fly_gather_records(const int32_t *col_dev, const float *w_dev, int64_t n_w, const int32_t *ids_dev, int64_t n,
                       void *records_dev, void *stream);

/* The resting trajectory of training (chessfly/brain.py:238-252: the network with no position, one column) and
 * the drive the rows of each light-cone step get from outside the cone, k_t = (W c_{t-1} + b -
 * A_t c_{t-1}[R_{t-1}])[R_t], which is the sum over the edges whose presynaptic neuron lies outside R_{t-1}.
 *
 * fly_rest_forward, one step over W's CSR (crow, pre, w; rows are postsynaptic neurons, n of them):
 *   full[i] = sum_e w_e x2[pre_e].x + bias[i], outside[i] = sum_e w_e x2[pre_e].y + bias[i],
 *   c_next[i] = lerp(c_prev[i], clamp(full[i], 0, h_max), alpha[i]) (torch.lerp's formula),
 *   x2_next[i] = {c_next[i], member[i] ? 0 : c_next[i]}  (the next step's pairs; member = this step's rows).
 * x2 holds n float pairs {c_{t-1}, c_{t-1} outside R_{t-1}}, or NULL for the first step (c_0 = 0, no edge terms);
 * c_prev NULL means 0; member NULL means no rows.  alpha = sigmoid(alpha_logit).
 *
 * fly_rest_backward, that step's elementwise gradients per neuron: from gc = dL/dc_t (NULL: 0), gk = dL/dk_t and
 * gp = dL/dp_t with p_t = c_{t-1}[R_t] (|R_t| each, NULL: 0; pos[i] = i's place in R_t or -1), writes
 * g2[i] = {dL/dfull_i, dL/doutside_i} and gc_prev = dL/dc_{t-1} through the lerp and p_t, and adds to gbias and
 * galpha.
 *
 * fly_rest_products_backward, that step's products: gw[e] += g2[post_e] . x2[pre_e] over W, then
 * gc_prev[j] += sum over row j of W^T of w_e (g2[i].x + (member_prev[j] ? 0 : g2[i].y)) over W^T's work list
 * (t_rowptr / t_col / t_val, items / splits / partials as for fly_spmv_work; member_prev = R_{t-1}, NULL: none).
 * Row pointers are clamped and pair reads bounded, so a malformed structure gives wrong results, never an access
 * outside the arrays; n below 2^28. */
int fly_rest_forward(const int32_t *crow_dev, const int32_t *pre_dev, const float *w_dev, int64_t n, int64_t nnz,
                     const float *x2_dev, const float *bias_dev, const float *alpha_dev, const float *c_prev_dev,
                     float h_max, const uint8_t *member_dev, float *full_dev, float *outside_dev, float *c_next_dev,
                     float *x2_next_dev, void *stream);
int fly_rest_backward(const float *gc_dev, const int32_t *pos_dev, const float *gk_dev, const float *gp_dev,
                      const float *full_dev, const float *c_prev_dev, const float *alpha_dev, float h_max, int64_t n,
                      float *g2_dev, float *gc_prev_dev, float *gbias_dev, float *galpha_dev, void *stream);
int fly_rest_products_backward(const int32_t *crow_dev, const int32_t *pre_dev, int64_t n, int64_t nnz,
                               const float *g2_dev, const float *x2_dev, float *gw_dev, const int32_t *t_rowptr_dev,
                               const int32_t *t_col_dev, const float *t_val_dev, const uint8_t *member_prev_dev,
                               const int32_t *items_dev, int64_t n_items, const int32_t *splits_dev,
                               int64_t n_splits, float *partials_dev, int64_t n_slots, float *gc_prev_dev,
                               void *stream);

/* y (+)= A x for one column over a work list: items_dev (n_items, 4) int32 {row, first non-zero, count, slot}
 * cover every row, each row's segments in order (as chessfly.brain.backward_work builds them for a row
 * pointer: a row's first segment has slot -1, its later ones slots >= 0).  An item with slot < 0 writes
 * y[row * ldy] (adds to it when accumulate != 0); slot >= 0 writes partials_dev[slot], and splits_dev
 * (n_splits, 4) int32 {row, first slot, slot count, 0} then add those slots to y[row * ldy] in slot order.
 * Long rows (a transposed connectome's out-degrees run to thousands) thus spread over several waves and the
 * sums stay deterministic.
 * x[col * ldx].  Row pointers are clamped into [0, nnz] and items into their rows, so a malformed structure
 * gives wrong results, never an access outside the arrays. */
int fly_spmv_work(const int32_t *rowptr_dev, const int32_t *col_dev, const float *val_dev, int64_t nnz,
                  int64_t nrows, int64_t ncols, const float *x_dev, int64_t ldx, float *y_dev, int64_t ldy,
                  int32_t accumulate, const int32_t *items_dev, int64_t n_items, const int32_t *splits_dev,
                  int64_t n_splits, float *partials_dev, int64_t n_slots, void *stream);

/* The backward of y = A h in one pass over A^T (CSR t_rowptr / t_col, values vals in that order, ids = each
 * non-zero's index in the weight vector): gh (ncols of A, ldgh) (+)= A^T gy and gw[ids[e]] += sum_b
 * gy[row_e, b] h[col_e, b].  Every gathered row of gy serves both.  nrows = rows of A^T (= rows of h),
 * ncols = columns of A^T (= rows of gy); nnz = non-zeros of A^T; n_w = entries of gw.  The batch must be a
 * multiple of 4 and the rows 16-byte aligned; ids distinct.  Row pointers are clamped into [0, nnz] and ids at
 * or past n_w skipped, so a malformed structure gives wrong results, never an access outside the arrays.
 *
 * items (null: one wave per row of A^T) is a work list of n_items int32 quadruples {row, first non-zero
 * within the row, count, slot}, 16-byte aligned, covering every non-zero once and every row's first non-zero
 * with a slot -1 item.  A slot -1 item writes gh[row]; an item with slot s in [0, n_slots) writes its share of
 * gh[row] to partials (n_slots, ldgh), and splits (n_splits quadruples {row, first slot, slot count, unused})
 * then adds each split row's slots to gh[row] in slot order.  Long rows of A^T can so run on several waves at
 * once with deterministic sums; the list's order is the waves' order (longest first keeps the tail short).
 * Items and splits are clamped like the row pointers.
 *
 * dots (NULL: one fused pass) is a workspace of n_dots >= ceil(batch / 64) * nnz floats.  With it the pass
 * runs chunk-major: every wave of one 64-column chunk of gy runs before the next chunk's, so the gathers share
 * that chunk's slice of gy in the caches.  Each non-zero's dot over a chunk is stored in dots, and a second
 * kernel adds the chunks in order into gw[ids[e]]; results stay deterministic.  Worth it for batches of more
 * than 64 columns.
 *
 * Either way gw is updated in A^T's order.  A caller that keeps gw in the transposed order of the whole
 * weight vector, with ids = each non-zero's position in that order, has ids that rise along the pass, so the
 * updates of gw stream instead of landing on random lines.  Replaces _SparseRecurrent.backward
 * (brain.py:79-99), whose grad_h is a cuSPARSE SpMM over W^T and whose grad_w a column-blocked SDDMM. */
int fly_transposed_backward(const int32_t *t_rowptr_dev, const int32_t *t_col_dev, const float *vals_dev,
                            const int32_t *ids_dev, int64_t nnz, int64_t nrows, int64_t ncols, const float *gy_dev,
                            int64_t ldgy, const float *h_dev, int64_t ldh, int64_t batch, float *gh_dev,
                            int64_t ldgh, int32_t accumulate, float *gw_dev, int64_t n_w, const int32_t *items_dev,
                            int64_t n_items, const int32_t *splits_dev, int64_t n_splits, float *partials_dev,
                            int64_t n_slots, float *dots_dev, int64_t n_dots, void *stream);

/* The same backward as a banded sweep of gy's rows: sweep = the tables of A^T's structure (fly_sweep_create over
 * t_rowptr / t_col, rows = columns of A), records_dev = A^T's nnz {column, value bits} pairs in its CSR order,
 * ids_dev = each non-zero's slot in gw (ids at or past n_w skipped).  gh (rows of A^T, ldgh) (+)= A^T gy, split
 * rows' pieces added in piece order; each record's dot with the row's own h over each 32-column chunk is kept in
 * the workspace and the chunks are added in order into gw[ids[e]], so results are deterministic.  The batch must be
 * a multiple of 4 and the rows of gy, h and gh 16-byte aligned.  workspace: fly_transposed_backward_swept_workspace
 * bytes, 256-byte aligned. */
size_t fly_transposed_backward_swept_workspace(const fly_sweep *sweep, int64_t batch);
int fly_transposed_backward_swept(const fly_sweep *sweep, const void *records_dev, int64_t nnz, const int32_t *ids_dev,
                                  const float *gy_dev, int64_t ldgy, const float *h_dev, int64_t ldh, int64_t batch,
                                  float *gh_dev, int64_t ldgh, int32_t accumulate, float *gw_dev, int64_t n_w,
                                  void *workspace_dev, size_t workspace_bytes, void *stream);

/* One recurrent step of training, the elementwise parts fused (brain.py:313-327 under autograd), float32,
 * one row of R_t per wave; rows are (rows, batch) with leading dimensions ld*:
 *   forward:  y = s + k[r] + (usrc[r] >= 0 ? u[usrc[r]] : 0)   (s = A_t h_{t-1} in s_y, or 0 when has_s == 0;
 *             y overwrites s_y), x = clamp(y, 0, h_max), p = prev[r] >= 0 ? hprev[prev[r]] : pdef[r],
 *             h = torch.lerp(p, x, alpha[r]).
 *   backward: from g = dL/dh:  gy = g alpha [0 <= y <= h_max];  gk[r] = sum_b gy;  ga[r] = sum_b g (x - p);
 *             gpdef[r] = sum_b g (1 - alpha) on rows not carried, else 0;  carried rows store g (1 - alpha)
 *             into ghprev[prev[r]] (the caller zeroes ghprev, then adds A_t^T gy with fly_spmm accumulate or
 *             fly_transposed_backward);
 *             input rows add gy to gu[usrc[r]] (distinct rows per step).
 * prev / usrc may be NULL (no carried rows / no input rows). */
int fly_train_step_forward(int64_t rows, int64_t batch, float *s_y_dev, int64_t lds, int32_t has_s,
                           const float *k_dev, const float *pdef_dev, const float *alpha_dev, const int32_t *prev_dev,
                           const int32_t *usrc_dev, const float *u_dev, int64_t ldu, const float *hprev_dev,
                           int64_t ldp, float h_max, float *h_dev, int64_t ldh, void *stream);
int fly_train_step_backward(int64_t rows, int64_t batch, const float *g_dev, int64_t ldg, const float *y_dev,
                            int64_t ldy, const float *pdef_dev, const float *alpha_dev, const int32_t *prev_dev,
                            const int32_t *usrc_dev, const float *hprev_dev, int64_t ldp, float h_max, float *gy_dev,
                            int64_t ldgy, float *gk_dev, float *ga_dev, float *gpdef_dev, float *gu_dev,
                            int64_t ldgu, float *ghprev_dev, int64_t ldgh, void *stream);

/* ---- measurement ------------------------------------------------------------------------------- */

/* Kernel classes timed by the profiler. */
enum fly_kernel_class {
    FLY_K_STATE_STEP = 0,   /* the fused SpMM + update step */
    FLY_K_ENCODER = 1,      /* encoder GEMM */
    FLY_K_HEAD = 2,         /* head GEMMs and logit assembly */
    FLY_K_OTHER = 3,        /* output gather, bias add, zero fill, the training products */
    FLY_K_CLASSES = 4
};
/* While enabled, every launch of the forward entry points is bracketed by HIP events on its stream (no
 * synchronisation is added).  Enabling (on = 1) clears the counters; on = 0 stops recording. */
int fly_profile_enable(int32_t on);
/* Waits for the recorded events and returns, per kernel class, the summed milliseconds and the number of
 * launches (arrays of FLY_K_CLASSES entries; either may be NULL). */
int fly_profile_read(double *ms, int64_t *launches);
/* Waits for the recorded events and returns the number of launches recorded; the first min(that, cap) get their
 * kernel class and milliseconds, in launch order (either array may be NULL).  -1 on error. */
int64_t fly_profile_launches(int32_t *cls, double *ms, int64_t cap);

/* ---- tuning (for sweeps; defaults are the measured best) --------------------------------------- */
/* Defaults for objects created afterwards: a plan, dense plan or fly_sweep captures the tuning current at its
 * creation, so plans built under different tuning each keep their own; the training products and
 * fly_evaluator_download read it at each call.  Set and read under a lock.
 * key "vec": elements per lane of the state step kernel (0 = automatic); "tiles": batch tiles swept
 * row-major (0 = automatic, 1 = all column chunks of a row back to back); "unroll": non-zeros each wave
 * gathers per iteration (8, 16 or 32; 0 = automatic); "nt_store": 1 writes the new state with non-temporal
 * stores; "groups": lane groups per wave that gather different non-zeros (1, 2, 4, 8; 0 = automatic);
 * "rows_mode": 1 gives each lane group its own row, -1 never, 0 for steps with short rows; "rows_vec":
 * half-state elements per lane of those row slots (8 = 16 bytes, 16 = 32 bytes; 0 = automatic); "spmm_groups":
 * lane groups of fly_spmm on 16-byte lanes (2, 4, 8; 0 = automatic); "gemm_tile": workgroup tile of the dense
 * maps (1 = 64 x 64, 2 = 128 x 64, 3 = 128 x 128, or 10 TM + TN for 32 TM x 32 TN with TM in {2, 3, 4} and TN in
 * {2, 4, 5}; 0 = automatic); "step_lds": bytes of LDS each state-step workgroup reserves, which caps the
 * workgroups a CU runs at once (0 = none); "download_blocks": workgroups of fly_evaluator_download when its call
 * passes 0 (0 = 16); "swept": -1 keeps the long-row steps on the grouped kernel instead of the banded sweep, 1
 * sweeps every step with a matrix whatever its size (small graphs in tests), 0 = the size rule; "sweep_bands":
 * source bands of the sweep, 3 or 4 (0 = 4); "sweep_order": -1 lets the swept waves take their rows in the initial
 * order instead of the searched one (0); "sweep_grid": workgroups of a swept step (0: one per CU), which sets the rows
 * each wave owns; "sweep_piece": split rows longer than this many non-zeros into pieces of at most this many (0: 3 x
 * the mean + 10); "sweep_deal": 1 deals the rows out to the waves by work always, -1 never (0: where the index order
 * leaves a workgroup over 5% above the mean work); "sweep_paired": 1 makes every swept wave
 * that owns over 24 rows walk two rows per pass (0, -1: one); "sweep_slots": 3 makes swept waves take their
 * rows in passes of 3 slots (0: 6 when a wave owns over 24 rows); "sweep_pipe": the next four rounds' gathers in
 * flight during the sums, 0 in passes of 3 slots, 1 also of 6, -1 never; "sweep_last_sync": 1 makes a swept
 * workgroup's waves also meet after a chunk's last band (0: they go on to the epilogue at once); "nt_load": 1 reads
 * the carried state with non-temporal loads.  Every selectable shape computes the same function. */
int fly_set_tuning(const char *key, int64_t value);
/* The current default of a tuning key (as fly_set_tuning left it). */
int fly_get_tuning(const char *key, int64_t *value);

#ifdef __cplusplus
}
#endif

#endif /* FLYEVAL_H */
