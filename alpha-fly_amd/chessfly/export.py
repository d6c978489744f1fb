"""The browser-engine export of a network (scripts/export_web.py:20-60): the effective synapse weights in CSR
order, the neuron constants, the encoder columns the network reads, the heads and the normaliser, as
little-endian binaries in chunks of at most 24 MiB plus a JSON manifest.

    export_web(net, out_dir)            write the export of a FlyChessNet
    read_web_export(out_dir)            the manifest and every tensor as a numpy array
    net_from_web_export(out_dir, ...)   a FlyChessNet that evaluates exactly the exported weights

Tensor names, kinds and shapes are the reference's, so its JavaScript engine and its manifests read these
files and the other way round:

    values      f16  (E,)          sign * w0 * exp(log_gain), CSR (post, pre) order
    crow        u32  (N+1,)        CSR row pointer
    col         u24  (3E,) bytes   presynaptic index, 3 little-endian bytes each
    bias, alpha f32  (N,)          alpha = sigmoid(alpha_logit)
    in_idx, out_idx  u32
    encoder_wT  f16  (n_base, n_in)    encoder.weight[:, :n_base] transposed
    encoder_b   f32
    norm_mean, norm_std   f32      norm_std = sqrt(var + eps)
    policy_w    f16  (moves, n_out);  policy_b, from_w, from_b, to_w, to_b, value_w, value_b  f32
"""

from __future__ import annotations

import json
import os

import numpy as np
import pandas as pd
import torch

from .connectome import Connectome
from .encoding import N_BASE

CHUNK = 24 * 2 ** 20
KINDS = {"f16": "<f2", "f32": "<f4", "u32": "<u4", "u24": "u1"}


def chunk_files(name: str, nbytes: int, chunk: int = CHUNK) -> list[str]:
    """File names of a tensor of `nbytes` bytes split into chunks (export_web.py:27-33; one file even when
    empty)."""
    return [f"weights/{name}.{i}.bin" for i in range(max(1, -(-nbytes // chunk)))]


def u24_bytes(col: np.ndarray) -> np.ndarray:
    """Indices below 2^24 as 3 little-endian bytes each (export_web.py:41)."""
    col = np.asarray(col, dtype=np.uint32)
    if col.size and int(col.max()) >= 1 << 24:
        raise ValueError("u24 indices must be below 2^24")
    return (col[:, None] >> np.array([0, 8, 16], dtype=np.uint32)).astype(np.uint8).reshape(-1)


def from_u24(raw: np.ndarray) -> np.ndarray:
    b = np.asarray(raw, dtype=np.uint32).reshape(-1, 3)
    return b[:, 0] | (b[:, 1] << 8) | (b[:, 2] << 16)


def export_web(net, out_dir: str, tests: list | None = None, checkpoint: str = "", chunk: int = CHUNK) -> dict:
    """Write the export of `net` (a FlyChessNet) to out_dir/manifest.json and out_dir/weights/*.bin and
    return the manifest.  `tests`, when given, is stored as the manifest's test positions."""
    brain, cfg = net.brain, net.cfg
    os.makedirs(os.path.join(out_dir, "weights"), exist_ok=True)
    manifest = {"neurons": brain.n, "edges": int(brain.pre.numel()), "steps": cfg.steps, "h_max": brain.h_max,
                "input_gain": cfg.input_gain, "n_base": N_BASE, "norm_eps": net.norm.eps, "norm_clip": net.norm.clip,
                "checkpoint": checkpoint, "tensors": {}}

    def put(name: str, arr: np.ndarray, kind: str) -> None:
        arr = np.ascontiguousarray(arr)
        raw = arr.tobytes()
        files = chunk_files(name, len(raw), chunk)
        for i, f in enumerate(files):
            with open(os.path.join(out_dir, f), "wb") as fh:
                fh.write(raw[i * chunk:(i + 1) * chunk])
        manifest["tensors"][name] = {"kind": kind, "shape": list(arr.shape), "files": files, "bytes": len(raw)}

    f32 = lambda t: t.detach().float().cpu().numpy()
    with torch.no_grad():
        put("values", f32(brain.sign * brain.w0 * torch.exp(brain.log_gain)).astype("<f2"), "f16")
        put("crow", brain.crow.cpu().numpy().astype("<u4"), "u32")
        put("col", u24_bytes(brain.pre.cpu().numpy()), "u24")
        put("bias", f32(brain.bias).astype("<f4"), "f32")
        put("alpha", f32(torch.sigmoid(brain.alpha_logit)).astype("<f4"), "f32")
        put("in_idx", net.in_idx.cpu().numpy().astype("<u4"), "u32")
        put("out_idx", net.out_idx.cpu().numpy().astype("<u4"), "u32")
        put("encoder_wT", f32(net.encoder.weight[:, :N_BASE].T.contiguous()).astype("<f2"), "f16")
        put("encoder_b", f32(net.encoder.bias).astype("<f4"), "f32")
        put("norm_mean", f32(net.norm.mean).astype("<f4"), "f32")
        put("norm_std", f32((net.norm.var + net.norm.eps).sqrt()).astype("<f4"), "f32")
        put("policy_w", f32(net.policy.weight).astype("<f2"), "f16")
        for name, t in (("policy_b", net.policy.bias), ("from_w", net.policy_from.weight),
                        ("from_b", net.policy_from.bias), ("to_w", net.policy_to.weight), ("to_b", net.policy_to.bias),
                        ("value_w", net.value.weight), ("value_b", net.value.bias)):
            put(name, f32(t).astype("<f4"), "f32")
    if tests is not None:
        manifest["tests"] = tests
    with open(os.path.join(out_dir, "manifest.json"), "w") as fh:
        json.dump(manifest, fh)
    return manifest


def read_web_export(out_dir: str) -> tuple[dict, dict]:
    """(manifest, {name: numpy array}) of an export; u24 tensors come back as uint32 indices.  Raises
    FileNotFoundError naming the missing chunk files when the export is incomplete."""
    with open(os.path.join(out_dir, "manifest.json")) as fh:
        manifest = json.load(fh)
    missing = [f for t in manifest["tensors"].values() for f in t["files"]
               if not os.path.exists(os.path.join(out_dir, f))]
    if missing:
        raise FileNotFoundError(f"incomplete export {out_dir}: missing {missing}")
    arrays = {}
    for name, t in manifest["tensors"].items():
        raw = b"".join(open(os.path.join(out_dir, f), "rb").read() for f in t["files"])
        if len(raw) != t["bytes"]:
            raise ValueError(f"{name}: {len(raw)} bytes on disk, {t['bytes']} in the manifest")
        a = np.frombuffer(raw, dtype=KINDS[t["kind"]]).reshape(t["shape"])
        arrays[name] = from_u24(a) if t["kind"] == "u24" else a
    return manifest, arrays


def net_from_web_export(out_dir: str, device="cuda"):
    """A FlyChessNet whose forward is the exported network: W = the exported values (w0 = |w|, sign = sign(w),
    log_gain = 0), alpha_logit = logit(alpha), the normaliser's var = norm_std^2 - eps."""
    from .model import FlyChessNet, ModelConfig
    m, a = read_web_export(out_dir)
    n, e = int(m["neurons"]), int(m["edges"])
    crow = a["crow"].astype(np.int64)
    if crow.shape != (n + 1,) or int(crow[-1]) != e or np.any(np.diff(crow) < 0):
        raise ValueError("crow does not describe a CSR matrix of the manifest's size")
    post = np.repeat(np.arange(n, dtype=np.int64), np.diff(crow))
    pre = a["col"].astype(np.int64)
    w = a["values"].astype(np.float32)
    flow = np.full(n, "intrinsic", dtype=object)
    flow[a["in_idx"]] = "afferent"
    flow[a["out_idx"]] = "efferent"
    neurons = pd.DataFrame({"root_id": np.arange(n), "super_class": flow, "cell_type": "", "nt": "", "flow": flow})
    sign = np.where(w < 0, -1.0, 1.0).astype(np.float32)
    conn = Connectome(neurons, torch.as_tensor(pre), torch.as_tensor(post), torch.as_tensor(np.abs(w)),
                      torch.as_tensor(sign))
    cfg = ModelConfig(steps=int(m["steps"]), input_gain=float(m["input_gain"]), weight_scale=1.0)
    net = FlyChessNet(conn, cfg)
    if not (np.array_equal(net.in_idx.numpy(), a["in_idx"]) and np.array_equal(net.out_idx.numpy(), a["out_idx"])):
        raise ValueError("in_idx / out_idx of the export are not sorted, unique index lists")
    t = lambda x: torch.as_tensor(np.asarray(x, dtype=np.float32))
    with torch.no_grad():
        brain = net.brain
        brain.w0.copy_(t(np.abs(w)))
        brain.sign.copy_(t(sign))
        brain.log_gain.zero_()
        brain.bias.copy_(t(a["bias"]))
        alpha = a["alpha"].astype(np.float64)
        brain.alpha_logit.copy_(t(np.log(alpha / (1.0 - alpha))))
        net.encoder.weight.zero_()
        net.encoder.weight[:, :int(m["n_base"])] = t(a["encoder_wT"]).T
        net.encoder.bias.copy_(t(a["encoder_b"]))
        net.norm.mean.copy_(t(a["norm_mean"]))
        std = a["norm_std"].astype(np.float64)
        net.norm.var.copy_(t(np.maximum(std * std - float(m["norm_eps"]), 0.0)))
        net.norm.eps, net.norm.clip = float(m["norm_eps"]), float(m["norm_clip"])
        net.norm.initialised.fill_(True)
        for name, layer in (("policy", net.policy), ("from", net.policy_from), ("to", net.policy_to),
                            ("value", net.value)):
            layer.weight.copy_(t(a[f"{name}_w"]))
            layer.bias.copy_(t(a[f"{name}_b"]))
    return net.to(device).eval()
