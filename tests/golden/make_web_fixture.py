"""Writes tests/golden/web_export_fixture.json from the browser export that ships with the reference
(docs/model/manifest.json and the weight chunks present beside it; values.0, col.0 and encoder_wT.0 are not
shipped).  Data only: the manifest's scalars and tensor table, and small byte samples of the real chunks with
the facts the reference's writer (scripts/export_web.py:20-60) fixes about them:

  crow.0.bin        u32 LE, N+1 entries, non-decreasing, first 0, last = the manifest's edge count
  col.1.bin         u24 LE: the second 24 MiB chunk of 3-byte column indices, so it starts at entry 2^23;
                    entries below N and ascending within each CSR row
  encoder_wT.1.bin, policy_w.0.bin   f16 LE weights

Run from the repository root:  python tests/golden/make_web_fixture.py
"""
import hashlib
import json
import os

import numpy as np

SRC = "/root/reference/docs/model"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "web_export_fixture.json")


def blob(name):
    path = os.path.join(SRC, name)
    return open(path, "rb").read() if os.path.exists(path) else None


m = json.load(open(os.path.join(SRC, "manifest.json")))
fixture = {"scalars": {k: v for k, v in m.items() if k not in ("tensors", "tests")},
           "tensors": m["tensors"], "present": {}, "samples": {}}
for t in m["tensors"].values():
    for f in t["files"]:
        raw = blob(f)
        if raw is not None:
            fixture["present"][f] = {"bytes": len(raw), "sha256": hashlib.sha256(raw).hexdigest()}

crow_raw = blob("weights/crow.0.bin")
col1_raw = blob("weights/col.1.bin")
first = (24 * 2 ** 20) // 3                      # index of the first entry in col.1.bin
n_col = 1000
crow = np.frombuffer(crow_raw, "<u4")
row0 = int(np.searchsorted(crow, first, side="right")) - 1
row1 = int(np.searchsorted(crow, first + n_col, side="right"))
fixture["samples"]["crow_head"] = {"hex": crow_raw[:64].hex()}
fixture["samples"]["crow_tail"] = {"hex": crow_raw[-64:].hex()}
fixture["samples"]["crow_rows"] = {"first_row": row0, "values": crow[row0:row1 + 1].tolist()}
fixture["samples"]["col1_head"] = {"first_entry": first, "hex": col1_raw[:3 * n_col].hex()}
for name in ("weights/encoder_wT.1.bin", "weights/policy_w.0.bin"):    # 2 KiB from the middle (the first rows
    raw = blob(name)                                                     # are untrained zeros)
    mid = len(raw) // 2 // 2048 * 2048
    fixture["samples"][name] = {"offset": mid, "hex": raw[mid:mid + 2048].hex()}
json.dump(fixture, open(OUT, "w"), indent=1)
print(f"wrote {OUT}: {len(fixture['present'])} present chunk files")
