"""Writes tests/golden/*.json: integer fixtures of the full-scale synthetic graphs and their light cones,
computed by the CPU oracle (oracle/lightcone.py).  The GPU tests rebuild the same graphs from their seeds
and hold the device cone to these digests bit for bit.

    python tests/golden/make_golden.py        (about a minute on 8 cores)
"""

from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
for p in (REPO, os.path.join(REPO, "alpha-fly_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

from chessfly.synthetic import FULL, synthetic_connectome, synthetic_params  # noqa: E402
from oracle.lightcone import light_cone  # noqa: E402


def digest(a) -> str:
    return hashlib.sha256(np.ascontiguousarray(np.asarray(a, dtype="<i4")).tobytes()).hexdigest()


def fdigest(a) -> str:
    return hashlib.sha256(np.ascontiguousarray(np.asarray(a, dtype="<f4")).tobytes()).hexdigest()


def cone_record(cone) -> dict:
    """Per step: sizes and digests of R_t, A_t (crow, local column, edge id), the carried-row table
    (position in R_{t-1} or -1) and the input table (position in in_idx or -1); out_src (-1 if absent)."""
    steps = []
    for t in range(cone.steps + 1):
        rec = {"rows": len(cone.rows[t]), "rows_sha": digest(cone.rows[t])}
        if t >= 1:
            prev = np.where(cone.carried[t], cone.prev_row[t], -1)
            usrc = np.full(len(cone.rows[t]), -1, dtype=np.int64)
            usrc[cone.u_pos[t]] = cone.u_src[t]
            rec.update(prev_sha=digest(prev), usrc_sha=digest(usrc), carried=int(cone.carried[t].sum()),
                       fed=int(len(cone.u_pos[t])))
            op = cone.ops[t]
            if op is None:
                rec.update(op=False, nnz=0)
            else:
                rec.update(op=True, nnz=int(len(op.edges)), crow_sha=digest(op.crow), col_sha=digest(op.pre),
                           edge_sha=digest(op.edges))
        steps.append(rec)
    out_src = np.full(len(cone.out_idx), -1, dtype=np.int64)
    out_src[cone.out_pos] = cone.out_src
    return {"steps": steps, "edge_visits": int(cone.edge_visits), "out_src_sha": digest(out_src),
            "out_hit": int(len(cone.out_pos))}


def graph_record(conn) -> dict:
    return {"n": conn.n_neurons, "edges": conn.n_edges, "pre_sha": digest(conn.pre.numpy()),
            "post_sha": digest(conn.post.numpy()), "syn_sha": fdigest(conn.syn_count.numpy()),
            "sign_sha": fdigest(conn.sign.numpy()), "in_sha": digest(conn.nodes("afferent").numpy()),
            "out_sha": digest(conn.nodes("efferent").numpy())}


def main() -> None:
    conn = synthetic_connectome(FULL)
    params = synthetic_params(conn, seed=0)
    record = {"spec": FULL.__dict__, "global_scale": params.global_scale, "graphs": {}}
    for name, graph in (("synthetic", conn), ("shuffled", conn.shuffled(0))):
        in_idx, out_idx = graph.nodes("afferent").numpy(), graph.nodes("efferent").numpy()
        entry = graph_record(graph)
        entry["cones"] = {}
        for steps in (4, 6):
            cone = light_cone(graph.n_neurons, graph.pre.numpy(), graph.post.numpy(), in_idx, out_idx, steps)
            entry["cones"][str(steps)] = cone_record(cone)
            print(name, steps, [s["rows"] for s in entry["cones"][str(steps)]["steps"]],
                  [s.get("nnz", 0) for s in entry["cones"][str(steps)]["steps"]], flush=True)
        record["graphs"][name] = entry
    with open(os.path.join(HERE, "fullscale_cone.json"), "w") as f:
        json.dump(record, f, indent=1, sort_keys=True)


if __name__ == "__main__":
    main()
