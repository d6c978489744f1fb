"""Writes tests/golden/realdeg_fixture.npz and realdeg_fixture.json from the MaleCNS wiring data that ships with
the reference's browser export (docs/model/weights, written by scripts/export_web.py:29-60).  Data only:

  crow.0.bin      u32 LE, the CSR row pointer of W[post, pre] (N + 1 entries): its differences are the neurons'
                  in-degrees (synapse partners per postsynaptic neuron)
  in_idx.0.bin    u32 LE, the sorted sensory neuron ids the network's encoder drives
  out_idx.0.bin   u32 LE, the sorted output neuron ids its heads read

The fixture keeps the in-degree sequence (uint16; the largest is 9,193) and the two id sets as uint16 gaps
(first id, then differences; every gap is below 2^16), compressed, with the SHA-256 of each source file and of
each stored array, so a test can check the fixture against the numbers it was made from.  The partners of each
neuron are not in the export's shipped chunks (col.0.bin is missing), so a graph built from this fixture draws them
from a seed (chessfly.synthetic.degree_connectome).

Run from the repository root:  python tests/golden/make_realdeg_fixture.py
"""
import hashlib
import json
import os

import numpy as np

SRC = "/root/reference/docs/model/weights"
HERE = os.path.dirname(os.path.abspath(__file__))


def raw(name: str) -> bytes:
    with open(os.path.join(SRC, name), "rb") as f:
        return f.read()


def sha(b: bytes) -> str:
    return hashlib.sha256(b).hexdigest()


crow_b, in_b, out_b = raw("crow.0.bin"), raw("in_idx.0.bin"), raw("out_idx.0.bin")
crow = np.frombuffer(crow_b, dtype="<u4").astype(np.int64)
in_idx = np.frombuffer(in_b, dtype="<u4").astype(np.int64)
out_idx = np.frombuffer(out_b, dtype="<u4").astype(np.int64)
assert crow[0] == 0 and np.all(np.diff(crow) >= 0)
deg = np.diff(crow)
assert deg.max() < 2 ** 16
gaps = {}
for name, ids in (("in_idx", in_idx), ("out_idx", out_idx)):
    g = np.diff(ids, prepend=0)
    assert np.all(g[1:] > 0) and g.max() < 2 ** 16, name
    gaps[name] = g.astype(np.uint16)
arrays = {"in_degree": deg.astype(np.uint16), "in_idx_gaps": gaps["in_idx"], "out_idx_gaps": gaps["out_idx"]}
np.savez_compressed(os.path.join(HERE, "realdeg_fixture.npz"), **arrays)
mean = deg.sum() / deg.size
limit = 4 * mean + 64
meta = {
    "source_sha256": {"crow.0.bin": sha(crow_b), "in_idx.0.bin": sha(in_b), "out_idx.0.bin": sha(out_b)},
    "array_sha256": {k: sha(v.tobytes()) for k, v in arrays.items()},
    "neurons": int(deg.size), "edges": int(crow[-1]), "sensory": int(in_idx.size), "outputs": int(out_idx.size),
    "in_degree": {"mean": round(float(mean), 4), "median": float(np.median(deg)), "max": int(deg.max()),
                  "zero": int((deg == 0).sum()), "over_4_mean_plus_64": int((deg > limit).sum()),
                  "edges_over_4_mean_plus_64": int(deg[deg > limit].sum())},
}
with open(os.path.join(HERE, "realdeg_fixture.json"), "w") as f:
    json.dump(meta, f, indent=1)
print(json.dumps(meta, indent=1))
