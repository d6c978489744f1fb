"""Oracle pins: independent fp64 brute force for tiny graphs.  TEST INFRASTRUCTURE ONLY.

These restate the *definitions* rather than the reference's code, so that a mistake in the restatements
in lightcone.py / forward.py (a dropped term, a wrong index, a transposed operand) shows up as a mismatch:

* dense_recurrence: h_{t+1} = (1 - alpha) h_t + alpha * min(relu(W h_t + b + u), H) with a dense W built by
  accumulating every edge (repeated pairs add up), from h_0 = 0 - the closed form the reference's own tests
  hold the sparse recurrence to (tests/test_core.py:22-27).
* hop_cone: the light-cone row sets from breadth-first hop distances, in pure Python: a neuron varies at step
  t iff its hop distance from the inputs is <= t-1, and still matters at step t iff its hop distance to the
  outputs is <= T-t (the LightCone docstring, chessfly/brain.py:126-135).
"""

from __future__ import annotations

from collections import deque

import numpy as np


def dense_matrix(n: int, pre, post, w) -> np.ndarray:
    W = np.zeros((n, n), dtype=np.float64)
    np.add.at(W, (np.asarray(post), np.asarray(pre)), np.asarray(w, dtype=np.float64))
    return W


def dense_recurrence(W: np.ndarray, bias, alpha, u: np.ndarray, steps: int, h_max: float | None = 10.0) -> np.ndarray:
    """u: (N, B) fp64.  Returns h_steps (N, B).  h_max None clamps only below (brain.py:178-182, 221)."""
    h_max = np.inf if h_max is None else h_max
    bias = np.asarray(bias, dtype=np.float64)[:, None]
    alpha = np.asarray(alpha, dtype=np.float64)[:, None]
    h = np.zeros_like(u, dtype=np.float64)
    for _ in range(steps):
        h = (1.0 - alpha) * h + alpha * np.minimum(np.maximum(W @ h + bias + u, 0.0), h_max)
    return h


def _hops(n: int, adjacency: list[list[int]], sources) -> list[float]:
    dist = [float("inf")] * n
    queue = deque()
    for s in sources:
        if dist[s] != 0:
            dist[s] = 0
            queue.append(s)
    while queue:
        v = queue.popleft()
        for nb in adjacency[v]:
            if dist[nb] == float("inf"):
                dist[nb] = dist[v] + 1
                queue.append(nb)
    return dist


def hop_cone(n: int, pre, post, in_idx, out_idx, steps: int) -> list[list[int]]:
    """R_0..R_T as sorted Python lists, from hop distances."""
    succ = [[] for _ in range(n)]
    pred = [[] for _ in range(n)]
    for p, q in zip(np.asarray(pre).tolist(), np.asarray(post).tolist()):
        succ[p].append(q)
        pred[q].append(p)
    from_in = _hops(n, succ, np.asarray(in_idx).tolist())
    to_out = _hops(n, pred, np.asarray(out_idx).tolist())
    rows = [[]]
    for t in range(1, steps + 1):
        rows.append([v for v in range(n) if from_in[v] <= t - 1 and to_out[v] <= steps - t])
    return rows


def brute_sub_matrix(pre, post, rows: list[int], cols: list[int]):
    """Edges of W[rows, cols] in W's edge order, with local (row, col) positions, by a direct scan."""
    row_at = {v: i for i, v in enumerate(rows)}
    col_at = {v: j for j, v in enumerate(cols)}
    edges, lrow, lcol = [], [], []
    for e, (p, q) in enumerate(zip(np.asarray(pre).tolist(), np.asarray(post).tolist())):
        if q in row_at and p in col_at:
            edges.append(e)
            lrow.append(row_at[q])
            lcol.append(col_at[p])
    return edges, lrow, lcol
