"""CPU checks that pin the training oracle (oracle/training.py) before it judges the device's gradients:
finite differences, a dense restatement, and the light cone against the full recurrence (the checks of
tests/test_core.py:30-44 and :309-338 in the reference)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import brain_arrays, random_params, tiny_connectome
from oracle import training as T
from oracle.forward import HeadArrays, model_forward
from oracle.lightcone import light_cone


def _leaves(b):
    for name in ("log_gain", "bias", "alpha_logit"):
        setattr(b, name, getattr(b, name).clone().requires_grad_(True))
    return b


def _grads(b, *extra):
    return [t.grad.clone() if t.grad is not None else torch.zeros_like(t)
            for t in (*extra, b.log_gain, b.bias, b.alpha_logit)]


def _zero(b, *extra):
    for t in (*extra, b.log_gain, b.bias, b.alpha_logit):
        t.grad = None


def test_sparse_recurrent_backward_matches_finite_differences():
    """Both gradients of y = A h, against torch.autograd.gradcheck in float64, on a CSR matrix with empty
    rows and columns and a repeated (row, column) pair."""
    rows = torch.tensor([0, 0, 1, 1, 1, 3, 3, 4])
    cols = torch.tensor([1, 1, 0, 2, 5, 3, 5, 0])
    op = T.Csr(T._crow(rows, 6), cols, rows, (6, 6))
    g = torch.Generator().manual_seed(0)
    h = torch.randn(6, 3, dtype=torch.double, generator=g, requires_grad=True)
    w = torch.randn(8, dtype=torch.double, generator=g, requires_grad=True)
    assert torch.autograd.gradcheck(lambda h_, w_: T.SparseRecurrent.apply(h_, w_, op), (h, w))


def test_literal_gradients_match_the_dense_recurrence():
    conn = tiny_connectome()
    b = _leaves(brain_arrays(conn, 3.0, *random_params(conn, 1), dtype=torch.double))
    u = torch.rand(4, conn.n_neurons, dtype=torch.double, requires_grad=True)
    target = torch.rand(4, conn.n_neurons, dtype=torch.double)
    results = []
    for fn in (lambda: T.literal_grad(b, u.T.contiguous(), 5).T, lambda: T.dense_literal(b, u, 5)):
        _zero(b, u)
        out = fn()
        ((out - target) ** 2).sum().backward()
        results.append([out.detach()] + _grads(b, u))
    for a, c in zip(*results):
        assert c.abs().sum() > 0
        torch.testing.assert_close(a, c, rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("steps", [1, 2, 4, 6])
def test_light_cone_gradients_equal_the_full_recurrence(steps):
    conn = tiny_connectome(120, 700, seed=3)
    b = _leaves(brain_arrays(conn, 3.0, *random_params(conn, 4), dtype=torch.double))
    in_idx, out_idx = torch.arange(0, 9), torch.arange(100, 120)
    cone = light_cone(conn.n_neurons, conn.pre.numpy(), conn.post.numpy(), in_idx.numpy(), out_idx.numpy(), steps)
    u_in = torch.randn(9, 5, dtype=torch.double, requires_grad=True)
    target = torch.randn(20, 5, dtype=torch.double)
    results = []
    for mode in ("full", "cone"):
        _zero(b, u_in)
        if mode == "full":
            u = torch.zeros(conn.n_neurons, 5, dtype=torch.double).index_add(0, in_idx, u_in)
            out = T.literal_grad(b, u, steps)[out_idx]
        else:
            out = T.cone_grad(b, cone, u_in)
        ((out - target) ** 2).sum().backward()
        results.append([out.detach()] + _grads(b, u_in))
    for a, c in zip(*results):
        torch.testing.assert_close(a, c, rtol=1e-9, atol=1e-11)
    assert steps == 1 or results[0][2].abs().sum() > 0     # one step never uses W: it multiplies a zero state


def test_model_forward_under_autograd_equals_the_pinned_forward():
    """model_grad (layers, autograd) computes the same logits as the forward oracle's float64 path."""
    conn = tiny_connectome(60, 600, seed=2)
    n = conn.n_neurons
    b = brain_arrays(conn, 3.0, *random_params(conn, 5), dtype=torch.double)
    in_idx, out_idx = torch.arange(0, 12), torch.arange(40, 60)
    cone = light_cone(n, conn.pre.numpy(), conn.post.numpy(), in_idx.numpy(), out_idx.numpy(), 4)
    rng = np.random.default_rng(0)
    d = lambda *s: torch.as_tensor(rng.normal(0, 0.3, s))
    moves = 50
    hp = HeadArrays(d(12, 30), d(12), 5.0, 24, d(moves, 20), d(moves), d(64, 20), d(64), d(64, 20), d(64), d(3, 20),
                    d(3), torch.as_tensor(rng.integers(0, 64, moves)), torch.as_tensor(rng.integers(0, 64, moves)),
                    d(20) * 0.1, 1.0 + d(20).abs())
    x = torch.as_tensor((rng.random((7, 30)) < 0.3).astype(np.float64))
    lg, wd = T.model_grad(hp, b, cone, x)
    rl, rw = model_forward(b, hp, cone, x, mode="f64")
    torch.testing.assert_close(lg, rl.to(lg.dtype), rtol=1e-10, atol=1e-12)
    torch.testing.assert_close(wd, rw.to(wd.dtype), rtol=1e-10, atol=1e-12)
