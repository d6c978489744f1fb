/*
 * flyprobe.h - measurement probes for bench.py (libflyprobe.so).  Not part of the evaluator's ABI
 * (include/flyeval.h) and not loaded by it: the library exists to put a ceiling beside the state step's time.
 *
 * Every entry point returns 0 on success and 1 on a bad argument or a HIP error, with a message from
 * flyprobe_last_error().  Pointers are device pointers; launches go on `stream`.
 */
#ifndef FLYPROBE_H
#define FLYPROBE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

const char *flyprobe_last_error(void);

/* pairs (nnz) = {col[q], bits of val[q]}: a plan matrix (fly_plan_matrix) packed back into the 8-byte records
 * the state step streams. */
int flyprobe_pack(const int32_t *col_dev, const float *val_dev, int64_t nnz, void *pairs_dev, void *stream);

/* The banded-sweep tables the evaluator builds for a step (its builder, build_sweep), from the step matrix (rowptr
 * nrows+1, pairs nnz) over prev_rows source rows: cfg[7] = {bands (3 or 4), paired (the order searched for two rows per
 * pass), workgroups (0: one per CU), force (sweep whatever the size), piece (0: automatic), search (0: the initial
 * order), deal (0: where the index order is unbalanced, 1 always, -1 never)}, as the evaluator derives them from its
 * tuning.  *sweep = NULL where the evaluator would not sweep the matrix, by the same rule.  Synchronises.
 * flyprobe_sweep_destroy frees it. */
int flyprobe_sweep_create(const int32_t *rowptr_dev, const void *pairs_dev, int64_t nrows, int64_t nnz,
                          int64_t prev_rows, const int32_t *cfg, void **sweep, void *stream);
int flyprobe_sweep_destroy(void *sweep);
/* The tables of a sweep handle, as the swept kernel reads them: info[7] = {positions, pieces, split rows, rows per
 * wave, bands, workgroups, paired}; range ((rows + pieces) x 2 bands), order (positions), split (split rows) and
 * split_ptr (split rows + 1) copied to the given device buffers (NULL skips one). */
int flyprobe_sweep_read(const void *sweep, int64_t *info, int32_t *range_dev, int32_t *order_dev, int32_t *split_dev,
                        int32_t *split_ptr_dev, void *stream);

/* The launch-time choice of the swept kernel that the replays mirror, as fly_set_tuning sets it for the
 * evaluator: "sweep_paired" (1 two rows per pass, -1 one, 0 by the state type).  Other keys are refused. */
int flyprobe_set_tuning(const char *key, int64_t value);

/* The replay of one state step's gather stream: the state step's own kernel (same launch shape, wave order,
 * pair loads and gathers, chosen by the same rule from nrows, nnz and the layout) with the FMAs replaced by an
 * XOR fold and no row constants, input, carried state, cross-lane sums or stores.  rowptr (nrows+1) and pairs
 * (nnz records) are A_t; xprev (prev_rows, ldx) the previous state, __half if state_f16 else float; batch
 * columns.  sweep (from flyprobe_sweep_create, or NULL): the replay of a swept step is the swept kernel's.  sink: at
 * least 1 KiB, written only if the folded bits hit one value. */
int flyprobe_replay_step(const int32_t *rowptr_dev, const void *pairs_dev, int64_t nrows, int64_t nnz,
                         const void *xprev_dev, int64_t prev_rows, int64_t ldx, int64_t batch, int32_t state_f16,
                         const void *sweep, void *sink_dev, void *stream);

/* params (nrows 32-byte row records) with zero constants and the given prev (position in R_{t-1}, -1: not carried)
 * and usrc (input row, -1: none), as fly_cone_step exports them: the row reads of a replay with I/O. */
int flyprobe_pack_params(const int32_t *prev_dev, const int32_t *usrc_dev, int64_t nrows, void *params_dev,
                         void *stream);

/* The replay with the step's row I/O: as flyprobe_replay_step, plus each row's constants, carried state and input
 * drive u (n_in, ldu float32, padded like the model forward's; NULL: none) read and the new state xout (nrows, ldx)
 * written, without the arithmetic of the sum.  The pieces of split rows store nothing and are not finished. */
int flyprobe_replay_step_io(const int32_t *rowptr_dev, const void *pairs_dev, const void *params_dev, int64_t nrows,
                            int64_t nnz, const void *xprev_dev, int64_t prev_rows, int64_t ldx, const float *u_dev,
                            int64_t n_in, int64_t ldu, void *xout_dev, int64_t batch, int32_t state_f16,
                            const void *sweep, void *stream);

/* Uniform-random row gathers in the state step's lane layout: n reads of read_bytes (128: 8 rows per wave
 * instruction; 64: 16 rows) at byte offset idx[e] * row_bytes (16 bytes per lane) of base (`bytes` long).
 * Offsets past `bytes` read zeros.  sink: 256 floats, written only if the data sum to a sentinel value. */
int flyprobe_random_gather(const void *base_dev, int64_t bytes, int64_t row_bytes, int64_t read_bytes,
                           const int32_t *idx_dev, int64_t n, float *sink_dev, void *stream);

/* The same reads with no index stream: read e of lane group g picks row h < rows by a hash of (g, e, seed), so the
 * rate is that of the reads alone.  (The index-streamed probe above waits for each index load from memory before
 * the reads issued after it can be used: vector memory counters retire in order.)  n rounded up to whole waves of
 * 1,024 reads per lane group. */
int flyprobe_hashed_gather(const void *base_dev, int64_t bytes, int64_t rows, int64_t row_bytes, int64_t read_bytes,
                           int64_t n, int64_t seed, float *sink_dev, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* FLYPROBE_H */
