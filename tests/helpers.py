"""Shared fixtures: tiny graphs, oracle array bundles and the repo paths."""

from __future__ import annotations

import os
import sys

import numpy as np
import pandas as pd
import torch

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "alpha-fly_amd")
for p in (REPO, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)

from chessfly.connectome import Connectome  # noqa: E402
from oracle.forward import BrainArrays, HeadArrays, normalised_weight  # noqa: E402


def tiny_connectome(n: int = 30, e: int = 200, seed: int = 0) -> Connectome:
    """The reference's test graph (tests/test_core.py:12-19): e distinct (post, pre) pairs drawn by torch's
    seeded randperm over the n*n grid (self-loops allowed), sign per presynaptic neuron +1 with probability
    0.6, the first 5 neurons afferent and the last 5 efferent, syn_count uniform in 1..19."""
    g = torch.Generator().manual_seed(seed)
    pairs = torch.randperm(n * n, generator=g)[:e].sort().values
    post, pre = pairs // n, pairs % n
    nt_sign = torch.where(torch.rand(n, generator=g) < 0.6, 1.0, -1.0)
    flow = ["afferent"] * 5 + ["intrinsic"] * (n - 10) + ["efferent"] * 5
    neurons = pd.DataFrame({"root_id": np.arange(n), "super_class": flow, "cell_type": "", "nt": "", "flow": flow})
    return Connectome(neurons, pre, post, torch.randint(1, 20, (e,), generator=g).float(), nt_sign[pre])


def brain_arrays(conn: Connectome, global_scale: float, log_gain, bias, alpha_logit, h_max: float = 10.0,
                 dtype=torch.float32) -> BrainArrays:
    """Oracle inputs from a Connectome and parameter arrays (w0 recomputed by the oracle's own formula)."""
    w0 = normalised_weight(conn.n_neurons, conn.post, conn.syn_count.to(torch.float32)) * global_scale
    t = lambda a: torch.as_tensor(np.asarray(a)).to(dtype)
    return BrainArrays(conn.n_neurons, conn.pre.clone(), conn.post.clone(), conn.sign.to(dtype), w0.to(dtype),
                       t(log_gain), t(bias), t(alpha_logit), h_max)


def head_arrays(maps, input_gain: float, n_base: int, move_from, move_to, n_out: int) -> HeadArrays:
    t = lambda a: torch.as_tensor(np.asarray(a, dtype=np.float32))
    return HeadArrays(t(maps.encoder_w), t(maps.encoder_b), input_gain, n_base,
                      t(maps.policy_w), t(maps.policy_b), t(maps.from_w), t(maps.from_b), t(maps.to_w), t(maps.to_b),
                      t(maps.value_w), t(maps.value_b), torch.as_tensor(move_from), torch.as_tensor(move_to),
                      torch.zeros(n_out), torch.ones(n_out))


def random_params(conn: Connectome, seed: int, gain_sd: float = 0.3, bias_mean: float = 0.1, bias_sd: float = 0.2,
                  alpha_sd: float = 1.0):
    rng = np.random.default_rng(seed)
    return (rng.normal(0, gain_sd, conn.n_edges).astype(np.float32),
            rng.normal(bias_mean, bias_sd, conn.n_neurons).astype(np.float32),
            rng.normal(0, alpha_sd, conn.n_neurons).astype(np.float32))


REALDEG_FIXTURE = os.path.join(REPO, "tests", "golden", "realdeg_fixture.npz")


def realdeg_connectome(seed: int = 0) -> Connectome:
    """The full-scale graph with the MaleCNS wiring's in-degree sequence and sensory / output sets (the committed
    fixture made by tests/golden/make_realdeg_fixture.py) and partners drawn from `seed`."""
    from chessfly.synthetic import degree_connectome
    f = np.load(REALDEG_FIXTURE)
    ids = lambda gaps: np.cumsum(gaps.astype(np.int64))
    return degree_connectome(f["in_degree"], ids(f["in_idx_gaps"]), ids(f["out_idx_gaps"]), seed=seed)
