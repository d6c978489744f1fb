"""Oracle: the light cone and its per-step sub-matrices, restated in numpy.  TEST INFRASTRUCTURE ONLY
(imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline; never by the product).

Follows chessfly/brain.py:126-173 (LightCone) and :102-123 (_SubMatrix).  Definitions:

  V_0 = {},  V_1 = inputs,  V_t = V_{t-1} + {post_e : pre_e in V_{t-1}}       (within t-1 hops of an input)
  D_T = outputs,  D_t = D_{t+1} + {pre_e : post_e in D_{t+1}}                 (within T-t hops of an output)
  R_t = sorted(V_t & D_t)                                                     (R_0 is empty)

Per step t = 1..T, with where_{t-1}[v] = position of v in R_{t-1} or -1:
  sub-matrix A_t = W[R_t, R_{t-1}] as the edges e (in W's edge order) with post_e in R_t and pre_e in
  R_{t-1}; its local row/column indices; crow by counting rows; None when R_{t-1} is empty.
  carried = where_{t-1}[R_t] >= 0; keep_next = nonzero(carried); keep_prev = where_{t-1}[R_t][carried];
  prev_row = max(where_{t-1}[R_t], 0); u_pos = rows of R_t that are inputs; u_src = their input position.
  out_pos = outputs present in R_T; out_src = their position in R_T.
All arrays are int64 (bool for carried), as the reference's torch tensors are.
"""

from __future__ import annotations

import dataclasses

import numpy as np


@dataclasses.dataclass
class SubMatrix:
    edges: np.ndarray          # global edge ids, increasing
    post: np.ndarray           # local row (position in R_t), non-decreasing
    pre: np.ndarray            # local column (position in R_{t-1})
    crow: np.ndarray           # len(R_t) + 1
    shape: tuple[int, int]


@dataclasses.dataclass
class Cone:
    steps: int
    rows: list                 # R_0 .. R_T
    ops: list                  # [None, A_1, ..., A_T]
    keep_next: list
    keep_prev: list
    carried: list
    prev_row: list
    u_pos: list
    u_src: list
    out_pos: np.ndarray
    out_src: np.ndarray
    out_idx: np.ndarray
    edge_visits: int


def _mask(n: int, idx: np.ndarray) -> np.ndarray:
    m = np.zeros(n, dtype=bool)
    m[idx] = True
    return m


def _positions(n: int, members: np.ndarray) -> np.ndarray:
    where = np.full(n, -1, dtype=np.int64)
    where[members] = np.arange(len(members), dtype=np.int64)
    return where


def reach_sets(n: int, pre: np.ndarray, post: np.ndarray, in_idx: np.ndarray, out_idx: np.ndarray, steps: int):
    """(V_0..V_T, D_0..D_T) as boolean masks."""
    forward = [np.zeros(n, dtype=bool), _mask(n, in_idx)]
    while len(forward) <= steps:
        last = forward[-1]
        grown = last.copy()
        grown[post[last[pre]]] = True
        forward.append(grown)
    backward = [None] * (steps + 1)
    backward[steps] = _mask(n, out_idx)
    for t in range(steps - 1, -1, -1):
        later = backward[t + 1]
        grown = later.copy()
        grown[pre[later[post]]] = True
        backward[t] = grown
    return forward[:steps + 1], backward


def sub_matrix(n: int, pre: np.ndarray, post: np.ndarray, rows: np.ndarray, cols: np.ndarray) -> SubMatrix:
    row_at, col_at = _positions(n, rows), _positions(n, cols)
    edges = np.flatnonzero((row_at[post] >= 0) & (col_at[pre] >= 0)).astype(np.int64)
    lpost, lpre = row_at[post[edges]], col_at[pre[edges]]
    crow = np.zeros(len(rows) + 1, dtype=np.int64)
    np.cumsum(np.bincount(lpost, minlength=len(rows)), out=crow[1:])
    return SubMatrix(edges, lpost, lpre, crow, (len(rows), len(cols)))


def light_cone(n: int, pre, post, in_idx, out_idx, steps: int, prune: bool = True) -> Cone:
    """prune=False keeps every neuron at every step t >= 1 (R_t = all, R_0 empty): the literal recurrence
    in the same bookkeeping."""
    pre = np.asarray(pre, dtype=np.int64)
    post = np.asarray(post, dtype=np.int64)
    in_idx = np.asarray(in_idx, dtype=np.int64)
    out_idx = np.asarray(out_idx, dtype=np.int64)
    if prune:
        fwd, bwd = reach_sets(n, pre, post, in_idx, out_idx, steps)
    else:
        fwd = [np.zeros(n, dtype=bool)] + [np.ones(n, dtype=bool) for _ in range(steps)]
        bwd = [np.ones(n, dtype=bool) for _ in range(steps + 1)]
    rows = [np.flatnonzero(fwd[t] & bwd[t]).astype(np.int64) for t in range(steps + 1)]
    in_at = _positions(n, in_idx)
    ops, keep_next, keep_prev, carried, prev_row, u_pos, u_src = ([None] for _ in range(7))
    for t in range(1, steps + 1):
        r_prev, r_next = rows[t - 1], rows[t]
        ops.append(sub_matrix(n, pre, post, r_next, r_prev) if len(r_prev) else None)
        where = _positions(n, r_prev)[r_next]
        is_carried = where >= 0
        keep_next.append(np.flatnonzero(is_carried).astype(np.int64))
        keep_prev.append(where[is_carried])
        carried.append(is_carried)
        prev_row.append(np.maximum(where, 0))
        fed = in_at[r_next]
        u_pos.append(np.flatnonzero(fed >= 0).astype(np.int64))
        u_src.append(fed[fed >= 0])
    last_at = _positions(n, rows[steps])[out_idx]
    out_pos = np.flatnonzero(last_at >= 0).astype(np.int64)
    visits = sum(len(op.edges) for op in ops if op is not None)
    return Cone(steps, rows, ops, keep_next, keep_prev, carried, prev_row, u_pos, u_src,
                out_pos, last_at[out_pos], out_idx, int(visits))
