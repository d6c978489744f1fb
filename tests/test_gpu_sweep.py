"""GPU parity of the banded sweep (k_state_step_swept and the finish kernel of split rows) against the CPU oracle on
small graphs, where the size rule alone would never sweep: the sweep_mode fixture (conftest.py) forces it and picks
the launch shapes, so the same oracle checks run through spread rows, passes of 6 and of 3 slots, several passes per
wave, paired passes, 3 bands, the unsearched order and rows split into pieces.  Also: a graph with the real
connectome's kind of in-degrees (neurons with no partners, hub neurons), the sweep tables shared by every weight
version of a cone, and plans that keep the tuning they were created under.

Tolerances as in test_gpu_configs.py: float32 within float32 round-off of the float64 oracle (2e-5); the float16
deviation path against the exact function within 2e-3 of the deviation's own scale."""

from __future__ import annotations

import warnings

import numpy as np
import pytest
import torch

from conftest import swept_steps
from helpers import brain_arrays, random_params, tiny_connectome

from oracle import brute, lightcone as L, forward as F

warnings.filterwarnings("ignore", message="Sparse CSR tensor support is in beta")
pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _rnn(conn, scale, lg, b, al, h_max=10.0):
    from chessfly.brain import ConnectomeRNN
    rnn = ConnectomeRNN(conn, global_scale=scale, h_max=h_max)
    with torch.no_grad():
        rnn.log_gain.copy_(torch.as_tensor(lg))
        rnn.bias.copy_(torch.as_tensor(b))
        rnn.alpha_logit.copy_(torch.as_tensor(al))
    return rnn.to(DEV)


def _cone(conn, in_idx, out_idx, steps):
    return L.light_cone(conn.n_neurons, conn.pre.numpy(), conn.post.numpy(), np.asarray(in_idx),
                        np.asarray(out_idx), steps)


def _medium(seed):
    from chessfly.synthetic import GraphSpec, synthetic_connectome
    return synthetic_connectome(GraphSpec(n=3000, edges=120_000, n_sensory=300, n_output=80, seed=seed))


def _heavy_tailed(seed):
    """3,000 neurons with in-degrees like the MaleCNS wiring's: LogNormal around 25, a tenth of the neurons with no
    partner at all, and hubs of 1,500, 900 and 400 partners (far past 3 x the mean + 10, so the tables split them)."""
    from chessfly.synthetic import degree_connectome
    rng = np.random.default_rng([seed, 77])
    n = 3000
    deg = np.minimum(np.rint(rng.lognormal(np.log(25.0), 1.0, n)), 600).astype(np.int64)
    deg[rng.choice(n, n // 10, replace=False)] = 0
    deg[[17, 1500, 2999]] = [1500, 900, 400]
    ids = rng.permutation(n)
    return degree_connectome(deg, np.sort(ids[:300]), np.sort(ids[300:380]), seed=seed)


def _forward_io_both(rnn, conn, ba, batch, steps, seed, mode):
    """forward_io in float32 and float16 against the oracle on `batch` boards; returns the float32 plan's swept
    steps."""
    from chessfly import _hip
    in_idx, out_idx = conn.nodes("afferent"), conn.nodes("efferent")
    u_in = torch.randn(len(in_idx), batch, generator=torch.Generator().manual_seed(seed))
    cone = _cone(conn, in_idx, out_idx, steps)
    ind, outd = in_idx.to(DEV), out_idx.to(DEV)
    with torch.no_grad():
        out32 = rnn.forward_io(u_in.to(DEV), ind, outd, steps)
        out16 = rnn.forward_io(u_in.half().to(DEV), ind, outd, steps)
        dcone = rnn.light_cone(ind, outd, steps)
        swept32 = swept_steps(rnn._cone_plan(dcone, _hip.MODE_F32).handle, steps)
        swept16 = swept_steps(rnn._cone_plan(dcone, _hip.MODE_DEVIATION_F16).handle, steps)
    exact = F.cone_f32(ba, cone, u_in.double(), steps).numpy()
    np.testing.assert_allclose(out32.cpu().numpy(), exact, rtol=2e-5, atol=2e-5 * max(np.abs(exact).max(), 1.0),
                               err_msg=f"float32 {mode} B={batch}")
    exact16 = F.cone_f32(ba, cone, u_in.half().double(), steps).numpy()
    dev_scale = np.abs(exact16 - F.cone_f32(ba, cone, torch.zeros_like(u_in).double(), steps).numpy()).max()
    err = np.abs(out16.cpu().numpy() - exact16).max()
    print(f"{mode} B={batch}: swept steps (t, positions, pieces, workgroups) float32 {swept32}, float16 {swept16}; "
          f"float16 error {err:.2e} of deviation scale {dev_scale:.2e}", flush=True)
    assert err < 2e-3 * max(dev_scale, 1e-3), (mode, batch, err, dev_scale)
    if mode != "auto":
        assert swept32 and swept16, "the forced sweep did not run"
    return swept32


@pytest.mark.parametrize("batch", [1, 5, 100, 130])
def test_swept_step_matches_the_oracle(sweep_mode, batch):
    """forward_io through the banded sweep on a 3,000-neuron graph (40 partners per neuron) in both state types, at
    batches that end inside a chunk (1, 5, 100) and that leave a part-filled last chunk (130)."""
    conn = _medium(2)
    lg, b, al = random_params(conn, 8, gain_sd=0.1)
    rnn = _rnn(conn, 4.0, lg, b, al)
    ba = brain_arrays(conn, 4.0, lg, b, al, dtype=torch.float64)
    swept = _forward_io_both(rnn, conn, ba, batch, 6, batch, sweep_mode)
    if sweep_mode == "swept-2wg-pieces":
        assert any(p > 0 for _, _, p, _ in swept), "no row was split into pieces"


@pytest.mark.parametrize("batch", [1, 5, 100, 130])
def test_swept_step_on_heavy_tailed_degrees(sweep_mode, batch):
    """A graph with neurons of no partner (empty rows of every step) and hubs of 400-1,500 partners, which the
    tables split into pieces: forward_io in both state types and the literal recurrence against the oracle."""
    conn = _heavy_tailed(3)
    lg, b, al = random_params(conn, 9, gain_sd=0.1)
    rnn = _rnn(conn, 4.0, lg, b, al)
    ba = brain_arrays(conn, 4.0, lg, b, al, dtype=torch.float64)
    deg = np.bincount(conn.post.numpy(), minlength=conn.n_neurons)
    assert (deg == 0).sum() >= 300 and deg.max() == 1500
    swept = _forward_io_both(rnn, conn, ba, batch, 6, 100 + batch, sweep_mode)
    if sweep_mode != "auto":
        assert any(p > 0 for _, _, p, _ in swept), "the hub rows were not split"
    u = torch.randn(conn.n_neurons, batch, generator=torch.Generator().manual_seed(batch))
    with torch.no_grad():
        h = rnn(u.clone().to(DEV), 4)
        full = rnn._full_plan()
    ref = F.literal(ba, u.double(), 4).numpy()
    np.testing.assert_allclose(h.cpu().numpy(), ref, rtol=2e-5, atol=2e-5 * np.abs(ref).max())
    if sweep_mode != "auto":
        info = swept_steps(full.handle, 1)
        assert info and info[0][2] > 0, ("the literal plan's hub rows were not split", info)


def test_swept_small_shuffled_graph_sums_repeats_and_self_loops(sweep_mode):
    """The shuffled control of the reference's test graph (repeated pairs and self-loops) through the forced sweep:
    forward_io in both dtypes and the literal recurrence against the dense float64 recurrence."""
    conn = tiny_connectome(80, 2000, 4).shuffled(3)
    lg, b, al = random_params(conn, 12, gain_sd=0.3, bias_sd=0.3)
    rnn = _rnn(conn, 3.0, lg, b, al)
    ba = brain_arrays(conn, 3.0, lg, b, al, dtype=torch.float64)
    W = brute.dense_matrix(conn.n_neurons, conn.pre.numpy(), conn.post.numpy(),
                           F.edge_weights(ba, torch.float64).numpy())
    alpha = 1 / (1 + np.exp(-al.astype(np.float64)))
    in_idx, out_idx = np.arange(0, 10), np.arange(60, 80)
    g = torch.Generator().manual_seed(4)
    for batch, steps in ((3, 2), (64, 4), (130, 6)):
        u_in = torch.randn(len(in_idx), batch, generator=g) * 0.5
        u = np.zeros((conn.n_neurons, batch))
        u[in_idx] = u_in.numpy()
        dense = brute.dense_recurrence(W, b.astype(np.float64), alpha, u, steps)
        ind, outd = torch.as_tensor(in_idx, device=DEV), torch.as_tensor(out_idx, device=DEV)
        with torch.no_grad():
            out32 = rnn.forward_io(u_in.to(DEV), ind, outd, steps)
            out16 = rnn.forward_io(u_in.half().to(DEV), ind, outd, steps)
            lit = rnn(torch.as_tensor(u, dtype=torch.float32).to(DEV), steps)
        np.testing.assert_allclose(out32.cpu().numpy(), dense[out_idx], rtol=2e-5, atol=2e-5)
        np.testing.assert_allclose(lit.cpu().numpy(), dense, rtol=2e-5, atol=2e-5)
        u16 = np.zeros_like(u)
        u16[in_idx] = u_in.half().double().numpy()
        exact16 = brute.dense_recurrence(W, b.astype(np.float64), alpha, u16, steps)[out_idx]
        rest = brute.dense_recurrence(W, b.astype(np.float64), alpha, np.zeros_like(u), steps)[out_idx]
        scale = max(np.abs(exact16 - rest).max(), 1e-3)
        err = np.abs(out16.cpu().numpy() - exact16).max()
        assert err < 2e-3 * scale, (sweep_mode, batch, steps, err, scale)


def test_second_weight_version_shares_the_sweep_tables(sweep_mode):
    """The sweep tables depend on the cone's structure only: a plan built for a second weight version reuses the
    first plan's tables (same tables identity in fly_plan_sweep_info), and its outputs equal, bit for bit, those of a
    plan built from scratch (a new network, a new cone) with the second version's weights."""
    from chessfly import _hip
    conn = _heavy_tailed(5)
    lg, b, al = random_params(conn, 31, gain_sd=0.1)
    rnn = _rnn(conn, 4.0, lg, b, al)
    in_idx, out_idx = conn.nodes("afferent").to(DEV), conn.nodes("efferent").to(DEV)
    u_in = torch.randn(len(in_idx), 96, generator=torch.Generator().manual_seed(2)).to(DEV)
    with torch.no_grad():
        for dtype, mode in ((torch.float16, _hip.MODE_DEVIATION_F16), (torch.float32, _hip.MODE_F32)):
            rnn.forward_io(u_in.to(dtype), in_idx, out_idx, 6)
            cone = rnn.light_cone(in_idx, out_idx, 6)
            first = swept_steps(rnn._cone_plan(cone, mode).handle, 6)
            first_ids = [_hip.sweep_info(rnn._cone_plan(cone, mode).handle, t)["tables"] for t in range(1, 7)]
            rnn.log_gain.add_(0.05)                          # a new weight version: a new plan on the same cone
            rnn.bias.mul_(0.9)
            second = rnn.forward_io(u_in.to(dtype), in_idx, out_idx, 6)
            plan2 = rnn._cone_plan(cone, mode)
            assert [_hip.sweep_info(plan2.handle, t)["tables"] for t in range(1, 7)] == first_ids
            fresh = _rnn(conn, 4.0, rnn.log_gain.detach().cpu().numpy(), rnn.bias.detach().cpu().numpy(), al)
            again = fresh.forward_io(u_in.to(dtype), in_idx, out_idx, 6)
            fresh_cone = fresh.light_cone(in_idx, out_idx, 6)
            fresh_ids = [_hip.sweep_info(fresh._cone_plan(fresh_cone, mode).handle, t)["tables"] for t in range(1, 7)]
            assert all(a != f for a, f in zip(first_ids, fresh_ids) if a), "the new cone built its own tables"
            print(f"{sweep_mode} {dtype}: swept steps {first}", flush=True)
            assert torch.equal(second, again), (sweep_mode, dtype)


def test_plans_keep_the_tuning_they_were_created_under():
    """Two networks on one graph: the first's plans are created under a forced sweep of 4 workgroups, the second's
    under the defaults afterwards; each keeps its own launch (fly_plan_sweep_info), whichever runs first, and both
    compute the oracle's function."""
    from chessfly import _hip
    conn = _medium(3)
    lg, b, al = random_params(conn, 14, gain_sd=0.1)
    ba = brain_arrays(conn, 4.0, lg, b, al, dtype=torch.float64)
    in_idx, out_idx = conn.nodes("afferent"), conn.nodes("efferent")
    ind, outd = in_idx.to(DEV), out_idx.to(DEV)
    u_in = torch.randn(len(in_idx), 64, generator=torch.Generator().manual_seed(7))
    exact = F.cone_f32(ba, _cone(conn, in_idx, out_idx, 6), u_in.double(), 6).numpy()
    a, d = _rnn(conn, 4.0, lg, b, al), _rnn(conn, 4.0, lg, b, al)
    _hip.set_tuning("swept", 1)
    _hip.set_tuning("sweep_grid", 4)
    try:
        with torch.no_grad():
            plan_a = a._cone_plan(a.light_cone(ind, outd, 6), _hip.MODE_F32)
    finally:
        _hip.set_tuning("swept", 0)
        _hip.set_tuning("sweep_grid", 0)
    with torch.no_grad():
        plan_d = d._cone_plan(d.light_cone(ind, outd, 6), _hip.MODE_F32)
        outs = [m.forward_io(u_in.to(DEV), ind, outd, 6) for m in (d, a, d)]
    sa, sd = swept_steps(plan_a.handle, 6), swept_steps(plan_d.handle, 6)
    print(f"forced plan: {sa}; default plan: {sd}", flush=True)
    assert sa and all(wg == 4 for *_, wg in sa) and not sd
    for o in outs:
        np.testing.assert_allclose(o.cpu().numpy(), exact, rtol=2e-5, atol=2e-5)
