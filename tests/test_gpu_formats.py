"""GPU test of the browser export (scripts/export_web.py:20-60): a network rebuilt from an export evaluates, on
the device, what the oracle computes from the exported arrays; and close to the network it came from (the
export stores W, the encoder and the policy in float16)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def test_network_from_an_export_matches_the_oracle(tmp_path):
    from chessfly.encoding import N_BASE
    from chessfly.export import export_web, net_from_web_export, read_web_export
    from chessfly.model import FlyChessNet, ModelConfig
    from chessfly.synthetic import GraphSpec, synthetic_boards, synthetic_connectome
    from oracle import forward as F
    from oracle.lightcone import light_cone
    conn = synthetic_connectome(GraphSpec(n=3000, edges=120_000, n_sensory=300, n_output=100, seed=8))
    torch.manual_seed(1)
    net = FlyChessNet(conn, ModelConfig(steps=4))
    with torch.no_grad():
        for p in net.parameters():
            p.add_(torch.randn_like(p) * 0.05)
        net.norm.mean.normal_(0, 0.2)
        net.norm.var.uniform_(0.5, 2.0)
    export_web(net, str(tmp_path))
    rebuilt = net_from_web_export(str(tmp_path), device=DEV)
    x = torch.as_tensor(synthetic_boards(24, seed=5), dtype=torch.float32)
    with torch.no_grad():
        logits, wdl = rebuilt(x.to(DEV))
        net32 = net.to(DEV).eval()
        net32.infer_dtype = torch.float32
        orig_logits, _ = net32(x.to(DEV))

    m, a = read_web_export(str(tmp_path))
    f = lambda v: torch.as_tensor(np.asarray(v, dtype=np.float32))
    w = a["values"].astype(np.float32)
    crow = a["crow"].astype(np.int64)
    post = torch.as_tensor(np.repeat(np.arange(m["neurons"]), np.diff(crow)))
    alpha = a["alpha"].astype(np.float64)
    ba = F.BrainArrays(m["neurons"], torch.as_tensor(a["col"].astype(np.int64)), post, f(np.where(w < 0, -1, 1)),
                       f(np.abs(w)), torch.zeros(len(w)), f(a["bias"]), f(np.log(alpha / (1 - alpha))))
    enc = np.zeros((len(a["in_idx"]), 967), np.float32)
    enc[:, :N_BASE] = a["encoder_wT"].astype(np.float32).T
    hp = F.HeadArrays(f(enc), f(a["encoder_b"]), m["input_gain"], N_BASE, f(a["policy_w"]), f(a["policy_b"]),
                      f(a["from_w"]), f(a["from_b"]), f(a["to_w"]), f(a["to_b"]), f(a["value_w"]), f(a["value_b"]),
                      rebuilt.move_from.cpu(), rebuilt.move_to.cpu(), f(a["norm_mean"]),
                      f(np.maximum(a["norm_std"].astype(np.float64) ** 2 - m["norm_eps"], 0)))
    cone = light_cone(m["neurons"], ba.pre.numpy(), post.numpy(), a["in_idx"].astype(np.int64),
                      a["out_idx"].astype(np.int64), m["steps"])
    ref_logits, ref_wdl = F.model_forward(ba, hp, cone, x, "f32")
    assert float((logits.cpu() - ref_logits).abs().max()) < 1e-3
    assert float((wdl.cpu() - ref_wdl).abs().max()) < 1e-3
    # the float16 storage of W, the encoder and the policy moves the logits only a little
    scale = float(orig_logits.abs().max())
    assert float((logits - orig_logits).abs().max()) < 2e-2 * scale
