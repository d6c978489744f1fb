"""Seeded synthetic connectome, network weights and boards with the sizes of the MaleCNS network.

The MaleCNS release is a network download, so the evaluator is exercised on a random graph with the same
neuron and synapse counts, built in the reference's own `Connectome` layout so it goes through the same
constructors (chessfly/connectome.py:54-95, chessfly/brain.py:176-199, chessfly/model.py:61-93):

* N = 166,700 neurons, about 10.5M directed edges.  Out-degrees are LogNormal(ln 63 - 1/2, 1) rounded and
  rescaled to the edge target; every edge's postsynaptic partner is uniform over the other neurons, so
  there are no self-loops, and repeated (post, pre) pairs are merged.
* syn_count ~ Geometric(1/4) on {1, 2, ...} (mean 4); the sign belongs to the presynaptic neuron and is +1
  with probability 0.6.
* 17,937 sensory ("afferent") and 2,333 output ("efferent") neurons, disjoint, drawn by the seed.
* log_gain ~ N(0, 0.1) per edge, bias ~ N(0.1, 0.05), alpha_logit ~ N(0, 1) per neuron, and a global weight
  scale chosen so that the spectral radius of the signed weight matrix is 0.9.
* Encoder (17,937 x 838 used columns), policy (4,168 x 2,333), from/to-square (64 x 2,333) and value
  (3 x 2,333) weights and biases ~ N(0, 1/sqrt(fan_in)); encoder columns 838..966 are zero.  The read-out
  normaliser keeps its fresh statistics (mean 0, variance 1).
* Boards: 838 base features in {0, 1} with exactly 40 ones, or a uniform 20..40 ones per board.

`degree_connectome` builds the same kind of graph around a given in-degree sequence and given sensory and
output sets (the MaleCNS wiring's, whose row pointer and id sets ship as weight data with the reference's
browser export): a heavy-tailed in-degree, with hub neurons of thousands of partners and neurons with none.

Everything is drawn with numpy's PCG64 generator from explicit seeds, so the same call gives the same
arrays on every machine with this numpy.
"""

from __future__ import annotations

import dataclasses
import functools

import numpy as np
import pandas as pd
import torch

from .connectome import Connectome
from .encoding import N_BASE, N_FEATURES, N_MOVES


@dataclasses.dataclass(frozen=True)
class GraphSpec:
    n: int = 166_700
    edges: int = 10_500_000
    n_sensory: int = 17_937
    n_output: int = 2_333
    mean_out: float = 63.0
    sigma: float = 1.0
    excitatory: float = 0.6
    syn_mean: float = 4.0
    seed: int = 0


FULL = GraphSpec()


def _flows(n: int, sensory: np.ndarray, output: np.ndarray) -> pd.DataFrame:
    flow = np.full(n, "intrinsic", dtype=object)
    flow[sensory] = "afferent"
    flow[output] = "efferent"
    sclass = np.full(n, "central", dtype=object)
    sclass[sensory] = "cb_sensory"
    sclass[output] = "cb_motor"
    return pd.DataFrame({"root_id": np.arange(n, dtype=np.int64), "super_class": sclass,
                         "cell_type": "", "nt": "", "flow": flow})


def synthetic_connectome(spec: GraphSpec = FULL) -> Connectome:
    """A random graph in CSR order of W[post, pre] (see the module docstring for the recipe)."""
    rng = np.random.default_rng([spec.seed, 0x5EED])
    n = spec.n
    raw = rng.lognormal(mean=np.log(spec.mean_out) - 0.5 * spec.sigma ** 2, sigma=spec.sigma, size=n)
    deg = np.clip(np.rint(raw * (spec.edges / raw.sum())), 0, n - 1).astype(np.int64)
    pre = np.repeat(np.arange(n, dtype=np.int64), deg)
    other = rng.integers(0, n - 1, size=pre.size, dtype=np.int64)
    post = other + (other >= pre)                          # uniform over the other n - 1 neurons
    key = np.unique(post * n + pre)                        # merge repeats; sorted = (post, pre) order
    post, pre = key // n, key % n
    syn = rng.geometric(1.0 / spec.syn_mean, size=key.size).astype(np.float32)
    nt_sign = np.where(rng.random(n) < spec.excitatory, 1.0, -1.0).astype(np.float32)
    chosen = rng.permutation(n)
    sensory = np.sort(chosen[:spec.n_sensory])
    output = np.sort(chosen[spec.n_sensory:spec.n_sensory + spec.n_output])
    return Connectome(_flows(n, sensory, output), torch.from_numpy(pre), torch.from_numpy(post),
                      torch.from_numpy(syn), torch.from_numpy(nt_sign[pre]))


def degree_connectome(in_degree: np.ndarray, sensory: np.ndarray, output: np.ndarray, seed: int = 0,
                      sigma: float = 1.0, excitatory: float = 0.6, syn_mean: float = 4.0) -> Connectome:
    """A graph in CSR order of W[post, pre] with the given in-degree per postsynaptic neuron and the given sorted
    sensory ("afferent") and output ("efferent") sets.  A neuron's presynaptic partners are distinct and never the
    neuron itself, each drawn with probability proportional to a per-neuron LogNormal(0, sigma) propensity (so
    out-degrees are heavy-tailed, as in synthetic_connectome); a draw that repeats a partner of the same neuron or
    hits the neuron itself is drawn again.  syn_count ~ Geometric(1 / syn_mean); the sign belongs to the
    presynaptic neuron (+1 with probability `excitatory`)."""
    rng = np.random.default_rng([seed, 0xDE6EE])
    deg = np.asarray(in_degree, dtype=np.int64)
    n = deg.size
    if deg.max(initial=0) >= n:
        raise ValueError("an in-degree reaches the neuron count: no distinct partners exist")
    cdf = np.cumsum(rng.lognormal(0.0, sigma, size=n))
    cdf /= cdf[-1]
    post = np.repeat(np.arange(n, dtype=np.int64), deg)
    pre = np.minimum(np.searchsorted(cdf, rng.random(post.size), side="right"), n - 1)
    for _ in range(1000):
        key = post * n + pre
        order = np.argsort(key, kind="stable")
        ks = key[order]
        bad = np.zeros(post.size, dtype=bool)
        bad[order[1:][ks[1:] == ks[:-1]]] = True           # a repeat of an earlier draw for the same neuron
        bad |= pre == post
        if not bad.any():
            break
        pre[bad] = np.minimum(np.searchsorted(cdf, rng.random(int(bad.sum())), side="right"), n - 1)
    else:
        raise RuntimeError("partner draws did not settle")
    key = np.sort(post * n + pre)                          # (post, pre) order
    post, pre = key // n, key % n
    syn = rng.geometric(1.0 / syn_mean, size=key.size).astype(np.float32)
    nt_sign = np.where(rng.random(n) < excitatory, 1.0, -1.0).astype(np.float32)
    sensory, output = np.sort(np.asarray(sensory, np.int64)), np.sort(np.asarray(output, np.int64))
    return Connectome(_flows(n, sensory, output), torch.from_numpy(pre), torch.from_numpy(post),
                      torch.from_numpy(syn), torch.from_numpy(nt_sign[pre]))


@dataclasses.dataclass
class NeuronParams:
    log_gain: np.ndarray      # (E,) float32
    bias: np.ndarray          # (N,) float32
    alpha_logit: np.ndarray   # (N,) float32
    global_scale: float


def spectral_radius(conn: Connectome, log_gain: np.ndarray, scale: float = 1.0, iters: int = 120) -> float:
    """Spectral radius of W = sign * weight * scale * exp(log_gain), by Gelfand's formula on a power
    iteration (||W^k v|| ** (1/k) over the last 40 products, which also settles for complex pairs)."""
    import scipy.sparse as sp
    n = conn.n_neurons
    w = (conn.sign.numpy().astype(np.float64) * conn.weight.numpy().astype(np.float64) * scale
         * np.exp(log_gain.astype(np.float64)))
    crow = np.zeros(n + 1, dtype=np.int64)
    np.cumsum(np.bincount(conn.post.numpy(), minlength=n), out=crow[1:])
    mat = sp.csr_matrix((w, conn.pre.numpy(), crow), shape=(n, n))
    v = np.ones(n) / np.sqrt(n)
    tail, log_growth = 40, 0.0
    for i in range(iters):
        v = mat @ v
        nv = float(np.linalg.norm(v))
        if nv == 0.0:
            return 0.0
        if i >= iters - tail:
            log_growth += np.log(nv)
        v /= nv
    return float(np.exp(log_growth / tail))


def synthetic_params(conn: Connectome, seed: int = 0, radius: float = 0.9) -> NeuronParams:
    rng = np.random.default_rng([seed, 0xB1A5])
    log_gain = rng.normal(0.0, 0.1, size=conn.n_edges).astype(np.float32)
    bias = rng.normal(0.1, 0.05, size=conn.n_neurons).astype(np.float32)
    alpha_logit = rng.normal(0.0, 1.0, size=conn.n_neurons).astype(np.float32)
    rho = spectral_radius(conn, log_gain)
    scale = float(f"{radius / rho:.6g}") if rho > 0 else 1.0
    return NeuronParams(log_gain, bias, alpha_logit, scale)


@dataclasses.dataclass
class DenseMaps:
    encoder_w: np.ndarray     # (n_in, N_FEATURES) float32, columns >= N_BASE zero
    encoder_b: np.ndarray
    policy_w: np.ndarray      # (N_MOVES, n_out)
    policy_b: np.ndarray
    from_w: np.ndarray        # (64, n_out)
    from_b: np.ndarray
    to_w: np.ndarray
    to_b: np.ndarray
    value_w: np.ndarray       # (3, n_out)
    value_b: np.ndarray


def synthetic_maps(n_in: int, n_out: int, seed: int = 0) -> DenseMaps:
    rng = np.random.default_rng([seed, 0xD3A5])

    def normal(shape, fan_in):
        return rng.normal(0.0, 1.0 / np.sqrt(fan_in), size=shape).astype(np.float32)

    enc = np.zeros((n_in, N_FEATURES), dtype=np.float32)
    enc[:, :N_BASE] = normal((n_in, N_BASE), N_BASE)
    return DenseMaps(enc, normal(n_in, N_BASE),
                     normal((N_MOVES, n_out), n_out), normal(N_MOVES, n_out),
                     normal((64, n_out), n_out), normal(64, n_out),
                     normal((64, n_out), n_out), normal(64, n_out),
                     normal((3, n_out), n_out), normal(3, n_out))


def synthetic_boards(batch: int, seed: int = 0, ones: int | tuple[int, int] = 40) -> np.ndarray:
    """(batch, N_FEATURES) float32 boards: `ones` of the N_BASE base features set to 1 (an int, or an
    inclusive (lo, hi) range drawn per board); the attack-plane columns are zero."""
    rng = np.random.default_rng([seed, 0xB0A2])
    if isinstance(ones, tuple):
        count = rng.integers(ones[0], ones[1] + 1, size=batch)
    else:
        count = np.full(batch, int(ones))
    rank = np.argsort(np.argsort(rng.random((batch, N_BASE)), axis=1), axis=1)
    x = np.zeros((batch, N_FEATURES), dtype=np.float32)
    x[:, :N_BASE] = rank < count[:, None]
    return x


@functools.lru_cache(maxsize=4)
def _cached_graph(spec: GraphSpec) -> Connectome:
    return synthetic_connectome(spec)


def synthetic_net(spec: GraphSpec = FULL, steps: int = 6, seed: int = 0, shuffled: bool = False,
                  device: str | torch.device = "cpu", graph: Connectome | None = None):
    """A FlyChessNet on the synthetic graph with every weight drawn from `seed` (returns the net and the
    Connectome it was built on).  `shuffled` builds the degree-preserving control graph instead; `graph` replaces
    the synthetic graph of `spec` (degree_connectome's, for example)."""
    from .model import FlyChessNet, ModelConfig
    conn = _cached_graph(spec) if graph is None else graph
    params = synthetic_params(conn, seed)
    cfg = ModelConfig(steps=steps, shuffled=shuffled, weight_scale=params.global_scale, input_gain=5.0, bias_init=0.1)
    net = FlyChessNet(conn, cfg)
    used = conn.shuffled() if shuffled else conn   # the same seed-0 control FlyChessNet built (same edge count)
    maps = synthetic_maps(len(net.in_idx), len(net.out_idx), seed)
    with torch.no_grad():
        net.brain.log_gain.copy_(torch.from_numpy(params.log_gain))
        net.brain.bias.copy_(torch.from_numpy(params.bias))
        net.brain.alpha_logit.copy_(torch.from_numpy(params.alpha_logit))
        net.encoder.weight.copy_(torch.from_numpy(maps.encoder_w))
        net.encoder.bias.copy_(torch.from_numpy(maps.encoder_b))
        net.policy.weight.copy_(torch.from_numpy(maps.policy_w))
        net.policy.bias.copy_(torch.from_numpy(maps.policy_b))
        net.policy_from.weight.copy_(torch.from_numpy(maps.from_w))
        net.policy_from.bias.copy_(torch.from_numpy(maps.from_b))
        net.policy_to.weight.copy_(torch.from_numpy(maps.to_w))
        net.policy_to.bias.copy_(torch.from_numpy(maps.to_b))
        net.value.weight.copy_(torch.from_numpy(maps.value_w))
        net.value.bias.copy_(torch.from_numpy(maps.value_b))
    return net.to(device).eval(), used


__all__ = ["GraphSpec", "FULL", "synthetic_connectome", "degree_connectome", "synthetic_params", "synthetic_maps", "synthetic_boards",
           "synthetic_net", "spectral_radius", "NeuronParams", "DenseMaps", "N_MOVES"]
