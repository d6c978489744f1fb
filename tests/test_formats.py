"""Formats around the evaluator (CPU): the browser export (scripts/export_web.py:20-60) against the manifest
and the real weight chunks that ship with the reference (fixture: tests/golden/web_export_fixture.json), the
checkpoint loader (chessfly/model.py:154-161) and the MaleCNS reader (chessfly/connectome.py:97-165) on
synthetic release files."""

from __future__ import annotations

import dataclasses
import json
import os

import numpy as np
import pandas as pd
import pytest
import torch

from helpers import REPO, tiny_connectome

FIXTURE = json.load(open(os.path.join(REPO, "tests", "golden", "web_export_fixture.json")))


def _net(conn=None, steps=3):
    from chessfly.model import FlyChessNet, ModelConfig
    torch.manual_seed(0)
    net = FlyChessNet(conn if conn is not None else tiny_connectome(60, 600, seed=2), ModelConfig(steps=steps))
    with torch.no_grad():
        for p in net.parameters():
            p.add_(torch.randn_like(p) * 0.1)
        net.norm.mean.normal_(0, 0.2)
        net.norm.var.uniform_(0.5, 2.0)
    return net


def test_chunking_reproduces_the_reference_file_lists():
    from chessfly.export import CHUNK, chunk_files
    for name, t in FIXTURE["tensors"].items():
        assert chunk_files(name, t["bytes"]) == t["files"], name
    for f, meta in FIXTURE["present"].items():          # each shipped chunk holds its share of the tensor
        name, i = f.split("/")[1].rsplit(".", 2)[0], int(f.rsplit(".", 2)[1])
        total = FIXTURE["tensors"][name]["bytes"]
        assert meta["bytes"] == min(CHUNK, total - i * CHUNK), f


def test_writer_schema_matches_the_reference_manifest(tmp_path):
    """Same scalar keys, tensor names in the same order, kinds, and the shape rules the reference's manifest
    obeys: values (E,), crow (N+1,), col (3E,) bytes, encoder_wT (n_base, n_in), policy_w (moves, n_out)."""
    from chessfly.export import export_web
    net = _net()
    m = export_web(net, str(tmp_path))
    ref = FIXTURE
    assert set(m) - {"tensors"} == set(ref["scalars"])
    assert list(m["tensors"]) == list(ref["tensors"])
    for name, t in m["tensors"].items():
        assert t["kind"] == ref["tensors"][name]["kind"], name
        assert t["bytes"] == int(np.prod(t["shape"])) * {"f16": 2, "f32": 4, "u32": 4, "u24": 1}[t["kind"]], name

    def rules(scalars, tensors):
        n, e = scalars["neurons"], scalars["edges"]
        n_in, n_out = tensors["in_idx"]["shape"][0], tensors["out_idx"]["shape"][0]
        moves = tensors["policy_w"]["shape"][0]
        want = {"values": [e], "crow": [n + 1], "col": [3 * e], "bias": [n], "alpha": [n], "encoder_wT":
                [scalars["n_base"], n_in], "encoder_b": [n_in], "norm_mean": [n_out], "norm_std": [n_out],
                "policy_w": [moves, n_out], "policy_b": [moves], "from_w": [64, n_out], "from_b": [64],
                "to_w": [64, n_out], "to_b": [64], "value_w": [3, n_out], "value_b": [3]}
        return {k: tensors[k]["shape"] for k in want} == want and moves == 4168
    assert rules(ref["scalars"], ref["tensors"])
    assert rules({k: v for k, v in m.items() if k != "tensors"}, m["tensors"])


def test_reader_decodes_the_reference_chunks():
    """The real row pointer, u24 columns and f16 weights, decoded as the reader decodes them."""
    from chessfly.export import from_u24
    s, sc = FIXTURE["samples"], FIXTURE["scalars"]
    head = np.frombuffer(bytes.fromhex(s["crow_head"]["hex"]), "<u4")
    tail = np.frombuffer(bytes.fromhex(s["crow_tail"]["hex"]), "<u4")
    assert head[0] == 0 and np.all(np.diff(head.astype(np.int64)) >= 0)
    assert int(tail[-1]) == sc["edges"] and np.all(np.diff(tail.astype(np.int64)) >= 0)
    cols = from_u24(np.frombuffer(bytes.fromhex(s["col1_head"]["hex"]), np.uint8))
    assert cols.max() < sc["neurons"]
    first = s["col1_head"]["first_entry"]
    crow = np.asarray(s["crow_rows"]["values"], np.int64)
    entries = np.arange(first, first + len(cols))
    rows = np.searchsorted(crow, entries, side="right") - 1
    for r in np.unique(rows):                       # CSR (post, pre) order: columns ascend inside a row
        assert np.all(np.diff(cols[rows == r].astype(np.int64)) > 0)
    for name in ("weights/encoder_wT.1.bin", "weights/policy_w.0.bin"):
        w = np.frombuffer(bytes.fromhex(s[name]["hex"]), "<f2").astype(np.float32)
        assert np.all(np.isfinite(w)) and np.abs(w).max() < 100 and np.abs(w).max() > 0


def test_export_round_trip_on_the_host(tmp_path):
    from chessfly.encoding import N_BASE
    from chessfly.export import export_web, read_web_export
    net = _net()
    export_web(net, str(tmp_path), chunk=512)               # small chunks: several files per tensor
    m, a = read_web_export(str(tmp_path))
    brain = net.brain
    assert len(m["tensors"]["col"]["files"]) > 1
    np.testing.assert_array_equal(a["crow"], brain.crow.numpy())
    np.testing.assert_array_equal(a["col"], brain.pre.numpy())
    w = (brain.sign * brain.w0 * torch.exp(brain.log_gain)).detach().numpy()
    np.testing.assert_array_equal(a["values"], w.astype(np.float16))
    np.testing.assert_array_equal(a["encoder_wT"], net.encoder.weight[:, :N_BASE].T.detach().numpy().astype(np.float16))
    np.testing.assert_allclose(a["alpha"], torch.sigmoid(brain.alpha_logit).detach().numpy(), rtol=1e-7)
    np.testing.assert_allclose(a["norm_std"], (net.norm.var + net.norm.eps).sqrt().numpy(), rtol=1e-7)
    os.remove(os.path.join(str(tmp_path), m["tensors"]["col"]["files"][1]))
    with pytest.raises(FileNotFoundError, match="col.1.bin"):
        read_web_export(str(tmp_path))


def test_load_net_reads_a_checkpoint(tmp_path):
    """A checkpoint dict {"config", "model", ...} through load_net, with torch.load(weights_only=True)."""
    from chessfly.model import load_net
    conn = tiny_connectome(60, 600, seed=2)
    net = _net(conn)
    path = os.path.join(str(tmp_path), "last.pt")
    torch.save({"config": dataclasses.asdict(net.cfg), "model": net.state_dict(), "iteration": 7,
                "opt": {"state": {}, "param_groups": [{"lr": 1e-3}]}}, path)
    got = load_net(path, device="cpu", conn=conn)
    assert not got.training
    for k, v in net.state_dict().items():
        assert torch.equal(got.state_dict()[k], v), k


def test_load_net_requires_the_connectome(tmp_path):
    """The reference's load_net parses the MaleCNS release when no graph is given; this package has no reader
    for it, so the graph must be passed (and nothing is read before that is checked)."""
    from chessfly.model import load_net
    with pytest.raises(ValueError, match="conn="):
        load_net(os.path.join(str(tmp_path), "missing.pt"), device="cpu")
