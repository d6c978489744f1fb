"""CPU tests of the drop-in host layer: module structure, state_dict keys and checkpoint loading behave as the
reference's chessfly.model / chessfly.brain (no GPU call is made)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import tiny_connectome

# The persistent state of the reference's FlyChessNet (chessfly/model.py:61-93, chessfly/brain.py:176-199): its
# parameters and the RunningNorm buffers; the wiring, index and move tables are non-persistent buffers.
REFERENCE_KEYS = {
    "brain.log_gain", "brain.bias", "brain.alpha_logit",
    "encoder.weight", "encoder.bias",
    "norm.mean", "norm.var", "norm.initialised",
    "policy.weight", "policy.bias", "value.weight", "value.bias",
    "policy_from.weight", "policy_from.bias", "policy_to.weight", "policy_to.bias",
}


def _net(**cfg):
    from chessfly.model import FlyChessNet, ModelConfig
    return FlyChessNet(tiny_connectome(60, 600), ModelConfig(steps=3, **cfg))


def test_state_dict_keys_and_shapes_match_the_reference():
    from chessfly.encoding import N_FEATURES, N_MOVES
    net = _net()
    sd = net.state_dict()
    assert set(sd) == REFERENCE_KEYS
    n_in, n_out = len(net.in_idx), len(net.out_idx)
    assert sd["encoder.weight"].shape == (n_in, N_FEATURES)
    assert sd["policy.weight"].shape == (N_MOVES, n_out) and sd["value.weight"].shape == (3, n_out)
    assert sd["brain.log_gain"].shape == (600,) and sd["brain.bias"].shape == (60,)
    # the reference's initialisation: zero heads except the policy bias, alpha = 0.5, bias = bias_init
    assert float(sd["policy.weight"].abs().sum()) == 0 and float(sd["value.weight"].abs().sum()) == 0
    assert float(sd["policy_from.weight"].abs().sum()) == 0 and float(sd["policy_to.bias"].abs().sum()) == 0
    torch.testing.assert_close(torch.sigmoid(sd["brain.alpha_logit"]), torch.full((60,), 0.5))
    torch.testing.assert_close(sd["brain.bias"], torch.full((60,), 0.1))
    assert net.infer_dtype == torch.float16


def test_in_and_out_neurons_follow_the_connectome_flows():
    net = _net()
    assert net.in_idx.tolist() == list(range(5)) and net.out_idx.tolist() == list(range(55, 60))
    w0 = tiny_connectome(60, 600).weight * 2.0
    torch.testing.assert_close(net.brain.w0, w0)
    crow = torch.zeros(61, dtype=torch.long)
    crow[1:] = torch.bincount(net.brain.post, minlength=60).cumsum(0)
    assert torch.equal(net.brain.crow, crow) and torch.equal(net.brain.crow32, crow.int())


def test_load_weights_accepts_old_checkpoints_and_rejects_incomplete_ones():
    """chessfly/model.py:141-151 and the checks of tests/test_core.py:394-415 / 418-428 that need no forward."""
    from chessfly.encoding import N_BASE
    from chessfly.model import load_weights
    net = _net()
    with torch.no_grad():
        net.policy.weight.normal_(0, 0.05)
    old = {k: v.clone() for k, v in net.state_dict().items() if not k.startswith(("policy_from.", "policy_to."))}
    fresh = _net()
    load_weights(fresh, old)                              # a checkpoint from before the from/to heads
    torch.testing.assert_close(fresh.policy.weight, net.policy.weight)
    narrow = dict(old)
    narrow["encoder.weight"] = old["encoder.weight"][:, :N_BASE].clone()
    wide = _net(attack_planes=True)
    load_weights(wide, narrow)                            # a checkpoint from before the attack planes
    assert float(wide.encoder.weight[:, N_BASE:].abs().sum()) == 0
    with pytest.raises(RuntimeError):
        load_weights(fresh, {k: v for k, v in old.items() if k != "value.bias"})


def test_running_norm_modes():
    """RunningNorm (chessfly/model.py:37-58): statistics update only in training mode with B > 1."""
    from chessfly.model import RunningNorm
    norm = RunningNorm(4)
    r = torch.tensor([[1.0, 2.0, 3.0, 40.0], [3.0, 2.0, 1.0, 0.0]])
    norm.eval()
    torch.testing.assert_close(norm(r), ((r - 0) / (1 + 1e-8) ** 0.5).clamp(-8, 8))
    norm.train()
    norm(r)
    torch.testing.assert_close(norm.mean, r.mean(0))
    torch.testing.assert_close(norm.var, r.var(0))
    norm(r[:1])                                           # B = 1 leaves the statistics alone
    torch.testing.assert_close(norm.mean, r.mean(0))
    assert bool(norm.initialised)


def test_expected_value():
    from chessfly.model import FlyChessNet
    wdl = torch.tensor([[2.0, 0.0, -1.0], [0.0, 0.0, 0.0]])
    p = np.exp(wdl.numpy()) / np.exp(wdl.numpy()).sum(1, keepdims=True)
    np.testing.assert_allclose(FlyChessNet.expected_value(wdl).numpy(), p[:, 0] - p[:, 2], rtol=1e-6)


def test_forward_refuses_host_tensors_in_every_mode():
    net = _net().eval()
    with torch.no_grad(), pytest.raises(RuntimeError, match="HIP device"):
        net(torch.zeros(2, 967))
    with pytest.raises(RuntimeError, match="HIP device"):
        net(torch.zeros(2, 967))                          # autograd on: the training path is device-only too
    net.train()
    with torch.no_grad(), pytest.raises(RuntimeError, match="HIP device"):
        net(torch.zeros(2, 967))
