"""GPU parity for the benchmark workloads and call paths beyond the headline forward: the shuffled control graph
(repeated pairs and self-loops summed), the unpruned float16-deviation and float32 forwards, 20-40-ones boards at
B = 256, the attack-plane encoder, the factorised policy head, unbounded activity (h_max=None), hub rows in a step
of short rows and the per-step export fly_plan_step, each against the CPU oracle (or, for the policy head, the
layer-by-layer path) through the C ABI.

Tolerances: float32 paths within float32 round-off of the float64 oracle (2e-5); full models within 1e-3 max-abs
of the oracle's float32 forward with the argmax equal; the float16 deviation path against the exact function
within 2e-3 of the deviation's own scale (the bound of the float16 path tests)."""

from __future__ import annotations

import warnings

import numpy as np
import pytest
import torch

from conftest import swept_steps
from helpers import brain_arrays, head_arrays, random_params, tiny_connectome

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


def _cone(conn, in_idx, out_idx, steps, prune=True):
    return L.light_cone(conn.n_neurons, conn.pre.numpy(), conn.post.numpy(), np.asarray(in_idx),
                        np.asarray(out_idx), steps, prune=prune)


def _full_oracle(conn, params_of, n_base=None, enc_w=None):
    """Oracle arrays of the full-scale synthetic network on `conn`, with the neuron parameters drawn for the
    graph `params_of` (the shuffled control keeps the parameters of the graph it was built from)."""
    from chessfly.encoding import N_BASE, move_squares
    from chessfly.synthetic import synthetic_maps, synthetic_params
    p = synthetic_params(params_of, seed=0)
    ba = brain_arrays(conn, p.global_scale, p.log_gain, p.bias, p.alpha_logit)
    in_idx, out_idx = conn.nodes("afferent"), conn.nodes("efferent")
    frm, to = move_squares()
    hp = head_arrays(synthetic_maps(len(in_idx), len(out_idx), 0), 5.0, n_base or N_BASE, frm, to, len(out_idx))
    if enc_w is not None:
        hp.enc_w = torch.as_tensor(enc_w)
    return ba, hp, _cone(conn, in_idx, out_idx, 6)


def _check_model(net, x, ref, boards, label, dtypes=(torch.float32, torch.float16)):
    """net(x) in each dtype: the first `boards` boards within 1e-3 of the oracle's (logits, wdl) with the argmax
    equal; returns the outputs per dtype."""
    ref_logits, ref_wdl = ref
    outs = {}
    try:
        for dtype in dtypes:
            net.infer_dtype = dtype
            with torch.no_grad():
                logits, wdl = net(x.to(DEV))
            torch.cuda.synchronize()
            outs[dtype] = (logits, wdl)
            dl = float((logits[:boards].cpu() - ref_logits).abs().max())
            dw = float((wdl[:boards].cpu() - ref_wdl).abs().max())
            print(f"{label} {dtype}: max |logit - oracle| {dl:.3e}, max |wdl - oracle| {dw:.3e}", flush=True)
            assert dl < 1e-3 and dw < 1e-3, (label, dtype, dl, dw)
            assert torch.equal(logits[:boards].cpu().argmax(1), ref_logits.argmax(1)), (label, dtype)
    finally:
        net.infer_dtype = torch.float16
    return outs


def _run(net, x, dtypes=(torch.float32, torch.float16)):
    """net(x) in each dtype: {dtype: (logits, wdl)} on the device."""
    outs = {}
    try:
        for dtype in dtypes:
            net.infer_dtype = dtype
            with torch.no_grad():
                outs[dtype] = net(x.to(DEV))
        torch.cuda.synchronize()
    finally:
        net.infer_dtype = torch.float16
    return outs


def _check_boards(outs, ref, label, rows=None):
    """Boards `rows` (all: None) of each dtype's output against the oracle's float32 forward of those boards (ref):
    max |logit diff| and max |wdl diff| below 1e-3 and the policy argmax equal on at least 99.9% of the boards (the
    north star's bar, at the reference's fp32 path); prints the figures."""
    ref_logits, ref_wdl = ref
    for dtype, (logits, wdl) in outs.items():
        lg, wd = logits.cpu(), wdl.cpu()
        if rows is not None:
            lg, wd = lg[rows], wd[rows]
        dl, dw = float((lg - ref_logits).abs().max()), float((wd - ref_wdl).abs().max())
        agree = (lg.argmax(1) == ref_logits.argmax(1)).float()
        print(f"{label} {dtype}: {lg.shape[0]} boards, max |logit - oracle| {dl:.3e}, max |wdl - oracle| {dw:.3e}, "
              f"argmax agrees on {int(agree.sum())}/{lg.shape[0]} ({float(agree.mean()):.4%})", flush=True)
        assert dl < 1e-3 and dw < 1e-3 and float(agree.mean()) >= 0.999, (label, dtype, dl, dw)


def _agree(outs, label):
    """float16 deviation vs float32 on every board: within 1e-3, argmax on >= 99.9% of the boards."""
    (l32, w32), (l16, w16) = outs[torch.float32], outs[torch.float16]
    dl, dw = float((l16 - l32).abs().max()), float((w16 - w32).abs().max())
    agree = float((l16.argmax(1) == l32.argmax(1)).float().mean())
    print(f"{label}: f16 vs f32 over {l16.shape[0]} boards: {dl:.3e} / {dw:.3e}, argmax {agree:.4%}", flush=True)
    assert dl < 1e-3 and dw < 1e-3 and agree >= 0.999, (label, dl, dw, agree)


# ---- the shuffled control graph (repeated (post, pre) pairs and self-loops) ----------------------------------

def test_shuffled_small_graph_sums_repeats_and_self_loops():
    """connectome.py:82-89 on the reference's test graph: the permutation creates repeated pairs and self-loops,
    which every product must sum.  forward (literal) and forward_io (both dtypes) against the dense float64
    recurrence of brute.dense_recurrence."""
    conn = tiny_connectome(80, 2000, 4).shuffled(3)
    key = conn.post * conn.n_neurons + conn.pre
    assert len(torch.unique(key)) < len(key) and bool((conn.pre == conn.post).any())
    lg, b, al = random_params(conn, 12, gain_sd=0.3, bias_sd=0.3)
    rnn = _rnn(conn, 3.0, lg, b, al)
    ba = brain_arrays(conn, 3.0, lg, b, al, dtype=torch.float64)
    W = brute.dense_matrix(conn.n_neurons, conn.pre.numpy(), conn.post.numpy(),
                           F.edge_weights(ba, torch.float64).numpy())
    alpha = 1 / (1 + np.exp(-al.astype(np.float64)))
    in_idx, out_idx = np.arange(0, 10), np.arange(60, 80)
    g = torch.Generator().manual_seed(4)
    for batch, steps in ((3, 1), (64, 4), (100, 6)):
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
        assert err < 2e-3 * scale, (batch, steps, err, scale)


def test_full_scale_shuffled_control_forward_matches_oracle():
    """The degree-preserving control graph at full scale (166,700 neurons, seed 0), B = 1120 boards through
    FlyChessNet in both dtypes: every board against the oracle's float32 forward on the shuffled arrays, and the
    float16 deviation path against float32 on all 1120."""
    from chessfly.synthetic import FULL, _cached_graph, synthetic_boards, synthetic_net
    net, conn_s = synthetic_net(steps=6, seed=0, shuffled=True, device=DEV)
    orig = _cached_graph(FULL)
    key = conn_s.post * conn_s.n_neurons + conn_s.pre
    repeats = conn_s.n_edges - len(torch.unique(key))
    loops = int((conn_s.pre == conn_s.post).sum())
    print(f"shuffled control: {repeats} repeated pairs, {loops} self-loops", flush=True)
    assert repeats > 0 and loops > 0
    ba, hp, cone = _full_oracle(conn_s, orig)
    x = torch.as_tensor(synthetic_boards(1120, seed=17))
    outs = _run(net, x)
    _check_boards(outs, F.model_forward(ba, hp, cone, x, "f32"), "shuffled B=1120")
    _agree(outs, "shuffled B=1120")
    del net
    torch.cuda.empty_cache()


# ---- pruning off: the float16 deviation path at B = 1120 and the float32 forward at B = 64 -------------------

def test_full_scale_unpruned_forward_matches_oracle(full_net):
    """light_cone_pruning = False computes every neuron at every step: the same function.  At B = 1120 in both
    dtypes (the unpruned float16 deviation forward), the first 32 boards against the oracle's float32 forward,
    float16 against float32 on all boards, and unpruned against pruned on the device."""
    from chessfly.synthetic import synthetic_boards
    net, conn = full_net
    ba, hp, cone = _full_oracle(conn, conn)
    x = torch.as_tensor(synthetic_boards(1120, seed=23))
    ref = F.model_forward(ba, hp, cone, x[:32], "f32")
    try:
        net.light_cone_pruning = False
        outs = _check_model(net, x, ref, 32, "unpruned B=1120")
        _agree(outs, "unpruned B=1120")
        net.light_cone_pruning = True
        pruned = _check_model(net, x, ref, 32, "pruned B=1120")
    finally:
        net.light_cone_pruning = True
    for dtype, tol in ((torch.float32, 5e-5), (torch.float16, 1e-3)):
        d = float((outs[dtype][0] - pruned[dtype][0]).abs().max())
        assert d < tol, (dtype, d)


def test_full_scale_float32_unpruned_b64_matches_literal_recurrence(full_net):
    """The float32 workload without the light cone at B = 64: FlyChessNet with pruning off against the oracle's
    literal recurrence (brain.py:211-223) over all 166,700 neurons, encoded and read out as model.py:95-105."""
    from chessfly.synthetic import synthetic_boards
    net, conn = full_net
    ba, hp, _ = _full_oracle(conn, conn)
    x = torch.as_tensor(synthetic_boards(64, seed=29))
    in_t, out_t = conn.nodes("afferent"), conn.nodes("efferent")
    u = torch.zeros(conn.n_neurons, 64).index_copy_(0, in_t, F.encode_input(hp, x, torch.float32))
    ref = F.heads(hp, F.norm(hp, F.literal(ba, u, 6)[out_t].T))
    try:
        net.light_cone_pruning = False
        _check_model(net, x, ref, 64, "literal B=64", dtypes=(torch.float32,))
    finally:
        net.light_cone_pruning = True


# ---- boards with 20-40 ones at B = 256 ----------------------------------------------------------------------

def test_full_scale_b256_boards_with_20_to_40_ones(full_net):
    """All 256 boards of the B = 256 workload (20-40 ones per board) against the oracle's float32 forward."""
    from chessfly.synthetic import synthetic_boards
    net, conn = full_net
    ba, hp, cone = _full_oracle(conn, conn)
    x = torch.as_tensor(synthetic_boards(256, seed=31, ones=(20, 40)))
    ones = x[:, :838].sum(1)
    assert int(ones.min()) >= 20 and int(ones.max()) <= 40 and int(ones.max()) > int(ones.min())
    outs = _run(net, x)
    _check_boards(outs, F.model_forward(ba, hp, cone, x, "f32"), "B=256 20-40 ones")
    _agree(outs, "B=256 20-40 ones")


def test_full_scale_b1120_every_board_matches_oracle(full_net):
    """The headline workload (light cone, B = 1120, 40 ones per board): every board, both dtypes, against the
    oracle's float32 forward, and the plan's long-row steps (3-5) on the banded sweep."""
    from chessfly import _hip
    from chessfly.synthetic import synthetic_boards
    net, conn = full_net
    ba, hp, cone = _full_oracle(conn, conn)
    x = torch.as_tensor(synthetic_boards(1120, seed=43))
    outs = _run(net, x)
    _check_boards(outs, F.model_forward(ba, hp, cone, x, "f32"), "B=1120")
    dcone = net.brain.light_cone(net.in_idx, net.out_idx, 6)
    for mode in (_hip.MODE_DEVIATION_F16, _hip.MODE_F32):
        assert [t for t, *_ in swept_steps(net.brain._cone_plan(dcone, mode).handle, 6)] == [3, 4, 5]


@pytest.mark.parametrize("batch,rows", [(4096, np.r_[0:32, 4064:4096]), (8192, np.r_[4096:4128, 8160:8192])])
def test_full_scale_large_batches_far_boards_match_oracle(full_net, batch, rows):
    """B = 4096 (its first and last 32 boards) and B = 8192, which runs as two column blocks of 4,096 boards in
    float16 and three in float32 (the state stays below 2 GiB): the second block's first and last 32 boards, both
    dtypes, against the oracle's float32 forward."""
    from chessfly.synthetic import synthetic_boards
    net, conn = full_net
    ba, hp, cone = _full_oracle(conn, conn)
    x = torch.as_tensor(synthetic_boards(batch, seed=47, ones=(20, 40)))
    outs = _run(net, x)
    _check_boards(outs, F.model_forward(ba, hp, cone, x[rows], "f32"), f"B={batch}", rows=rows)
    del outs
    torch.cuda.empty_cache()


def test_full_scale_real_in_degrees_forward_matches_oracle():
    """The network on the graph with the MaleCNS wiring's in-degrees (hub rows of up to 9,193 partners, 2,190 rows
    with none; partners seeded): its long-row steps sweep with the hub rows split into pieces, and B = 64 (every
    board) and B = 1120 (the first and last 64-board chunks) in both dtypes match the oracle's float32 forward."""
    from chessfly import _hip
    from chessfly.synthetic import synthetic_boards, synthetic_net
    from helpers import realdeg_connectome
    conn = realdeg_connectome()
    net, _ = synthetic_net(steps=6, seed=0, device=DEV, graph=conn)
    ba, hp, cone = _full_oracle(conn, conn)
    dcone = net.brain.light_cone(net.in_idx, net.out_idx, 6)
    x = torch.as_tensor(synthetic_boards(1120, seed=53))
    rows = np.r_[0:64, 1056:1120]
    outs = _run(net, x)
    _check_boards(outs, F.model_forward(ba, hp, cone, x[rows], "f32"), "real in-degrees B=1120", rows=rows)
    for mode in (_hip.MODE_DEVIATION_F16, _hip.MODE_F32):
        swept = swept_steps(net.brain._cone_plan(dcone, mode).handle, 6)
        print(f"real in-degrees, mode {mode}: swept steps (t, positions, pieces, workgroups) {swept}", flush=True)
        assert {3, 4} <= {t for t, *_ in swept} and all(p > 0 for t, _, p, _ in swept if t in (3, 4))
    x64 = x[:64]
    _check_boards(_run(net, x64), F.model_forward(ba, hp, cone, x64, "f32"), "real in-degrees B=64")
    del net
    torch.cuda.empty_cache()


# ---- attack planes: the encoder over all 967 feature columns -------------------------------------------------

def test_full_scale_attack_planes(full_net):
    """model.py:98-101: with attack_planes the encoder reads all 967 columns (k = 967 through the split-fp16
    GEMM); without them, columns 838..966 have no effect (test_core.py:474-489)."""
    from chessfly.encoding import N_BASE, N_FEATURES
    from chessfly.synthetic import synthetic_boards
    net, conn = full_net
    rng = np.random.default_rng(41)
    enc = net.encoder.weight.detach().cpu().numpy().copy()
    enc[:, N_BASE:] = rng.normal(0, 1 / np.sqrt(N_FEATURES), size=(enc.shape[0], N_FEATURES - N_BASE))
    x = torch.as_tensor(synthetic_boards(48, seed=37))
    x[:, N_BASE:] = torch.as_tensor((rng.random((48, N_FEATURES - N_BASE)) < 0.2).astype(np.float32))
    saved = net.encoder.weight.detach().clone()
    try:
        with torch.no_grad():
            net.encoder.weight.copy_(torch.as_tensor(enc))
        ba, hp_on, cone = _full_oracle(conn, conn, n_base=N_FEATURES, enc_w=enc)
        net.cfg.attack_planes = True
        ref_on = F.model_forward(ba, hp_on, cone, x, "f32")
        on = _check_model(net, x, ref_on, 48, "attack planes on")
        net.cfg.attack_planes = False
        _, hp_off, _ = _full_oracle(conn, conn, enc_w=enc)
        ref_off = F.model_forward(ba, hp_off, cone, x, "f32")
        off = _check_model(net, x, ref_off, 48, "attack planes off")
        x0 = x.clone()
        x0[:, N_BASE:] = 0
        for dtype in (torch.float32, torch.float16):
            net.infer_dtype = dtype
            with torch.no_grad():
                l0, w0 = net(x0.to(DEV))
            assert torch.equal(l0, off[dtype][0]) and torch.equal(w0, off[dtype][1]), dtype
            assert float((on[dtype][0] - off[dtype][0]).abs().max()) > 1e-2    # the planes do matter when on
    finally:
        net.cfg.attack_planes = False
        net.infer_dtype = torch.float16
        with torch.no_grad():
            net.encoder.weight.copy_(saved)


# ---- the factorised policy head ----------------------------------------------------------------------------------

def test_factorised_policy_head_is_a_no_op_until_trained():
    """model.py:80-93 (test_core.py:394-415): the from- and to-square heads start at zero, and a checkpoint from
    before them loads, so the fused forward's logits equal policy(norm(forward_io(...))).  Here the policy map is
    random (at its zero initialisation both sides would be the bias alone).  Float32: to float32 round-off of the
    layer-by-layer path; float16 deviation: within 1e-3 of it, the bound between the two precisions."""
    from chessfly.encoding import N_BASE, N_FEATURES
    from chessfly.model import FlyChessNet, ModelConfig, load_weights
    net = FlyChessNet(tiny_connectome(60, 600), ModelConfig(steps=3)).to(DEV).eval()
    old = {k: v for k, v in net.state_dict().items() if not k.startswith(("policy_from.", "policy_to."))}
    load_weights(net, old)                                  # a checkpoint from before the shared terms
    g = torch.Generator().manual_seed(5)
    with torch.no_grad():
        net.policy.weight.copy_(torch.randn(net.policy.weight.shape, generator=g) * 0.3)
        assert float(net.policy_from.weight.abs().sum() + net.policy_to.weight.abs().sum()) == 0
    x = torch.rand(3, N_FEATURES, generator=g).to(DEV)
    with torch.no_grad():
        enc = torch.nn.functional.linear(x[:, :N_BASE], net.encoder.weight[:, :N_BASE], net.encoder.bias)
        u_in = (enc * net.cfg.input_gain).T.contiguous()
        r = net.norm(net.brain.forward_io(u_in, net.in_idx, net.out_idx, 3).T.float())
        nn_only = net.policy(r)
        try:
            for dtype, tol in ((torch.float32, 1e-5), (torch.float16, 1e-3)):
                net.infer_dtype = dtype
                logits, _ = net(x)
                d = float((logits - nn_only).abs().max())
                print(f"{dtype}: max |fused - policy(norm(forward_io))| {d:.3e}", flush=True)
                torch.testing.assert_close(logits, nn_only, rtol=tol, atol=tol)
        finally:
            net.infer_dtype = torch.float16


# ---- h_max=None: no upper clamp --------------------------------------------------------------------------------

def _medium(seed):
    from chessfly.synthetic import GraphSpec, synthetic_connectome
    return synthetic_connectome(GraphSpec(n=3000, edges=120_000, n_sensory=300, n_output=80, seed=seed))


def test_unbounded_activity_literal_and_light_cone(sweep_core):
    """ConnectomeRNN(h_max=None) (brain.py:178-182, 221) with biases that drive activity past 10: the literal
    recurrence and forward_io in float32 against the float64 oracle, and the float16 deviation path against the
    exact function."""
    conn = _medium(4)
    lg, b, al = random_params(conn, 21, gain_sd=0.1, bias_mean=6.0, bias_sd=4.0)
    rnn = _rnn(conn, 3.0, lg, b, al, h_max=None)
    assert rnn.h_max is None
    ba = brain_arrays(conn, 3.0, lg, b, al, h_max=None, dtype=torch.float64)
    in_idx, out_idx = conn.nodes("afferent"), conn.nodes("efferent")
    g = torch.Generator().manual_seed(6)
    u = torch.randn(conn.n_neurons, 40, generator=g) * 2
    ref = F.literal(ba, u.double(), 5).numpy()
    assert ref.max() > 10.0
    with torch.no_grad():
        h = rnn(u.clone().to(DEV), 5)
    scale = np.abs(ref).max()
    np.testing.assert_allclose(h.cpu().numpy(), ref, rtol=2e-5, atol=2e-5 * scale)
    u_in = torch.randn(len(in_idx), 40, generator=g) * 2
    cone = _cone(conn, in_idx, out_idx, 6)
    exact = F.cone_f32(ba, cone, u_in.double(), 6).numpy()
    ind, outd = in_idx.to(DEV), out_idx.to(DEV)
    with torch.no_grad():
        out32 = rnn.forward_io(u_in.to(DEV), ind, outd, 6)
        out16 = rnn.forward_io(u_in.half().to(DEV), ind, outd, 6)
    np.testing.assert_allclose(out32.cpu().numpy(), exact, rtol=2e-5, atol=2e-5 * np.abs(exact).max())
    exact16 = F.cone_f32(ba, cone, u_in.half().double(), 6).numpy()
    dev_scale = np.abs(exact16 - F.cone_f32(ba, cone, torch.zeros_like(u_in).double(), 6).numpy()).max()
    err = np.abs(out16.cpu().numpy() - exact16).max()
    assert err < 2e-3 * max(dev_scale, 1e-3), (err, dev_scale)


def test_other_activity_bounds_literal_and_light_cone(sweep_core):
    """A bound other than 10 (the reference's fused kernel applies only at h_max == 10, brain.py:310; its general
    path clamps to any h_max, brain.py:321): activity pushed past h_max = 3.5 by the biases, the literal recurrence
    and forward_io in float32 against the float64 oracle, and the float16 deviation path against the exact
    function, as for h_max = None."""
    conn = _medium(5)
    lg, b, al = random_params(conn, 22, gain_sd=0.1, bias_mean=2.0, bias_sd=2.0)
    rnn = _rnn(conn, 3.0, lg, b, al, h_max=3.5)
    ba = brain_arrays(conn, 3.0, lg, b, al, h_max=3.5, dtype=torch.float64)
    in_idx, out_idx = conn.nodes("afferent"), conn.nodes("efferent")
    g = torch.Generator().manual_seed(8)
    u = torch.randn(conn.n_neurons, 40, generator=g) * 2
    ref = F.literal(ba, u.double(), 5).numpy()
    free = F.literal(brain_arrays(conn, 3.0, lg, b, al, h_max=None, dtype=torch.float64), u.double(), 5).numpy()
    assert ref.max() <= 3.5 and np.abs(ref - free).max() > 0.5      # the bound acts
    with torch.no_grad():
        h = rnn(u.clone().to(DEV), 5)
    np.testing.assert_allclose(h.cpu().numpy(), ref, rtol=2e-5, atol=2e-5 * np.abs(ref).max())
    u_in = torch.randn(len(in_idx), 40, generator=g) * 2
    cone = _cone(conn, in_idx, out_idx, 6)
    exact = F.cone_f32(ba, cone, u_in.double(), 6).numpy()
    ind, outd = in_idx.to(DEV), out_idx.to(DEV)
    with torch.no_grad():
        out32 = rnn.forward_io(u_in.to(DEV), ind, outd, 6)
        out16 = rnn.forward_io(u_in.half().to(DEV), ind, outd, 6)
    np.testing.assert_allclose(out32.cpu().numpy(), exact, rtol=2e-5, atol=2e-5 * np.abs(exact).max())
    exact16 = F.cone_f32(ba, cone, u_in.half().double(), 6).numpy()
    dev_scale = np.abs(exact16 - F.cone_f32(ba, cone, torch.zeros_like(u_in).double(), 6).numpy()).max()
    err = np.abs(out16.cpu().numpy() - exact16).max()
    assert err < 2e-3 * max(dev_scale, 1e-3), (err, dev_scale)


# ---- fly_plan_step: one step at a time ---------------------------------------------------------------------------

def _with_hubs(conn, n_hubs=3):
    """conn plus, into each of n_hubs intrinsic neurons, an edge from every sensory neuron it does not already hear
    (4 synapses, the presynaptic neuron's sign): rows of step 2 far longer than the mean."""
    from chessfly.connectome import Connectome
    n = conn.n_neurons
    pre, post = conn.pre.numpy(), conn.post.numpy()
    sens, hubs = conn.nodes("afferent").numpy(), conn.nodes("intrinsic").numpy()[:n_hubs]
    have = set(zip(post.tolist(), pre.tolist()))
    extra = np.array([(h, s_) for h in hubs for s_ in sens if (h, s_) not in have and h != s_], dtype=np.int64)
    sign_of = np.ones(n, dtype=np.float32)
    sign_of[pre] = conn.sign.numpy()
    new_post = np.concatenate([post, extra[:, 0]])
    new_pre = np.concatenate([pre, extra[:, 1]])
    syn = np.concatenate([conn.syn_count.numpy(), np.full(len(extra), 4.0, dtype=np.float32)])
    order = np.lexsort((new_pre, new_post))
    return Connectome(conn.neurons, torch.as_tensor(new_pre[order]), torch.as_tensor(new_post[order]),
                      torch.as_tensor(syn[order]), torch.as_tensor(sign_of[new_pre[order]]))


@pytest.mark.parametrize("batch", [100, 1120])
def test_hub_rows_in_a_step_of_short_rows_match_the_oracle(batch):
    """A step of short rows (row slots of 8 rows) holding a few rows far longer than the mean: three neurons hear
    every sensory neuron, so step 2's rows average a few non-zeros and theirs about 300, past the rule by which the
    plan runs their slots first for every chunk (more than max(64, 8 x the mean) non-zeros).  forward_io in
    float32 against the float64 oracle (2e-5) and the float16 deviation path against the exact function (the
    float16 bound of the other tests), at one chunk of columns and at several."""
    conn = _with_hubs(_medium(7))
    lg, b, al = random_params(conn, 23, gain_sd=0.1)
    rnn = _rnn(conn, 4.0, lg, b, al)
    ba = brain_arrays(conn, 4.0, lg, b, al, dtype=torch.float64)
    in_idx, out_idx = conn.nodes("afferent"), conn.nodes("efferent")
    cone = _cone(conn, in_idx, out_idx, 6)
    lens = np.diff(cone.ops[2].crow)
    assert lens.mean() < 16 and lens.max() > max(64, 8 * lens.sum() // len(lens)), (lens.mean(), lens.max())
    u_in = torch.randn(len(in_idx), batch, generator=torch.Generator().manual_seed(batch)) * 0.5
    exact = F.cone_f32(ba, cone, u_in.double(), 6).numpy()
    ind, outd = in_idx.to(DEV), out_idx.to(DEV)
    with torch.no_grad():
        out32 = rnn.forward_io(u_in.to(DEV), ind, outd, 6)
        out16 = rnn.forward_io(u_in.half().to(DEV), ind, outd, 6)
    np.testing.assert_allclose(out32.cpu().numpy(), exact, rtol=2e-5, atol=2e-5 * np.abs(exact).max())
    exact16 = F.cone_f32(ba, cone, u_in.half().double(), 6).numpy()
    dev_scale = np.abs(exact16 - F.cone_f32(ba, cone, torch.zeros_like(u_in).double(), 6).numpy()).max()
    err = np.abs(out16.cpu().numpy() - exact16).max()
    assert err < 2e-3 * max(dev_scale, 1e-3), (err, dev_scale)


def _plan_step(lib, _hip, plan, t, xprev, u, batch, xout):
    ws = _hip.workspace(lib.fly_plan_step_workspace(plan.handle, t, batch), torch.device(DEV))
    _hip.check(lib.fly_plan_step(plan.handle, t, _hip.ptr(xprev), xprev.stride(0) if xprev is not None else 0,
                                 _hip.ptr(u), u.stride(0) if u is not None else 0, batch, xout.data_ptr(),
                                 xout.stride(0), ws.data_ptr(), ws.numel(), _hip.stream(torch.device(DEV))),
               "fly_plan_step")


@pytest.mark.parametrize("batch", [5, 64, 100, 136])
def test_plan_step_matches_the_oracle_step_by_step(batch, sweep_core):
    """fly_plan_step (the per-step op of brain.py:273-277 / 310-313) fed the oracle's own state of R_{t-1}:
    float32 mode against f32_step in float64 (2e-5), deviation mode against deviation_step in float64 on the same
    float16-rounded inputs (one float16 rounding of the result), every step of a 6-step cone.  Batches of 5 and
    100 end inside a lane's columns, so no lane may read or write past the caller's columns (the banded sweep takes
    the float16 state only at batches in whole 8-column lanes, the float32 state at batches in whole 4-column
    lanes, under the forced sweep modes)."""
    from chessfly import _hip
    lib = _hip.load()
    conn = _medium(5)
    lg, b, al = random_params(conn, 22, gain_sd=0.1)
    rnn = _rnn(conn, 4.0, lg, b, al)
    ba = brain_arrays(conn, 4.0, lg, b, al, dtype=torch.float64)
    in_idx, out_idx = conn.nodes("afferent"), conn.nodes("efferent")
    steps = 6
    cone = _cone(conn, in_idx, out_idx, steps)
    dcone = rnn.light_cone(in_idx.to(DEV), out_idx.to(DEV), steps)
    u_in = torch.randn(len(in_idx), batch, generator=torch.Generator().manual_seed(batch)) * 0.5
    prep = F.prepare_f32(ba, cone, torch.float64)
    consts = F.deviation_constants(ba, cone, half=False)
    hs, ds = [], []
    F.run_f32(prep, steps, u_in.double(), states=hs)
    F.cone_half(ba, cone, u_in.half().double(), steps, half=False, states=ds)
    with torch.no_grad():
        p32 = rnn._cone_plan(dcone, _hip.MODE_F32)
        p16 = rnn._cone_plan(dcone, _hip.MODE_DEVIATION_F16)
    if sweep_core != "auto":
        assert swept_steps(p32.handle, steps) and swept_steps(p16.handle, steps), "the forced sweep has no tables"
    u32, u16 = u_in.to(DEV), u_in.half().to(DEV)
    for t in range(1, steps + 1):
        rows = len(cone.rows[t])
        # float32: the oracle's h_{t-1} rounded to float32 in, one step, against the float64 step on that input
        h_prev = hs[t - 2].float() if t > 1 else None
        out = torch.full((rows, batch), float("nan"), device=DEV)
        _plan_step(lib, _hip, p32, t, h_prev.to(DEV) if h_prev is not None else None, u32, batch, out)
        want = F.f32_step(prep, t, h_prev.double() if h_prev is not None else None, u_in.double())
        np.testing.assert_allclose(out.cpu().numpy(), want.numpy(), rtol=2e-5, atol=2e-5, err_msg=f"f32 t={t}")
        # deviation: d_{t-1} rounded to float16 in, against the exact algebra on the same inputs
        d_prev = ds[t - 2].half() if t > 1 else None
        out16 = torch.full((rows, batch), float("nan"), dtype=torch.float16, device=DEV)
        _plan_step(lib, _hip, p16, t, d_prev.to(DEV) if d_prev is not None else None, u16, batch, out16)
        want16 = F.deviation_step(consts, cone, t, d_prev.double() if d_prev is not None else None,
                                  u_in.half().double()).numpy()
        got16 = out16.double().cpu().numpy()
        assert np.isfinite(got16).all(), t
        np.testing.assert_allclose(got16, want16, rtol=1e-3, atol=1e-5, err_msg=f"deviation t={t}")


def test_plan_step_composes_to_forward_io_and_the_literal_step():
    """Steps 1..T through fly_plan_step give forward_io's outputs bit for bit (float32: the carried output rows
    are h_T itself), and a literal plan's one step from an arbitrary state matches literal_step."""
    from chessfly import _hip
    lib = _hip.load()
    conn = _medium(6)
    lg, b, al = random_params(conn, 23, gain_sd=0.1)
    rnn = _rnn(conn, 4.0, lg, b, al)
    in_idx, out_idx = conn.nodes("afferent").to(DEV), conn.nodes("efferent").to(DEV)
    batch, steps = 64, 6
    g = torch.Generator().manual_seed(2)
    u_in = (torch.randn(len(in_idx), batch, generator=g) * 0.5).to(DEV)
    with torch.no_grad():
        ref = rnn.forward_io(u_in, in_idx, out_idx, steps)
        cone = rnn.light_cone(in_idx, out_idx, steps)
        plan = rnn._cone_plan(cone, _hip.MODE_F32)
    h = None
    for t in range(1, steps + 1):
        nxt = torch.empty(cone.row_counts[t], batch, device=DEV)
        _plan_step(lib, _hip, plan, t, h, u_in, batch, nxt)
        h = nxt
    torch.testing.assert_close(ref[cone.out_pos], h[cone.out_src], rtol=0, atol=0)
    # the literal plan: h' = lerp(h, clamp(W h + drive, 0, H), alpha) from a random h
    ba = brain_arrays(conn, 4.0, lg, b, al, dtype=torch.float64)
    h0 = torch.rand(conn.n_neurons, 37, generator=g) * 3
    drive = torch.randn(conn.n_neurons, 37, generator=g) + torch.as_tensor(b)[:, None]
    with torch.no_grad():
        full = rnn._full_plan()
    out = torch.empty(conn.n_neurons, 37, device=DEV)
    _plan_step(lib, _hip, full, 1, h0.to(DEV), drive.to(DEV), 37, out)
    mat, alpha = F.literal_operands(ba, torch.float64)
    want = F.literal_step(ba, mat, alpha, h0.double(), drive.double())
    np.testing.assert_allclose(out.cpu().numpy(), want.numpy(), rtol=2e-5, atol=2e-5)


def test_plan_matrix_is_the_sub_matrix_with_its_weights():
    """fly_plan_matrix returns A_t as the steps read it: the cone's row pointer and local columns, and values
    w[edges] bit for bit (brain.py:267-268, 303: the cached per-step matrix)."""
    from chessfly import _hip
    lib = _hip.load()
    conn = _medium(7)
    lg, b, al = random_params(conn, 24, gain_sd=0.1)
    rnn = _rnn(conn, 4.0, lg, b, al)
    in_idx, out_idx = conn.nodes("afferent").to(DEV), conn.nodes("efferent").to(DEV)
    with torch.no_grad():
        cone = rnn.light_cone(in_idx, out_idx, 6)
        plan = rnn._cone_plan(cone, _hip.MODE_DEVIATION_F16)
        w = rnn.edge_weights()
    st = _hip.stream(torch.device(DEV))
    for t in range(1, 7):
        op = cone.ops[t]
        if op is None:
            continue
        nnz = cone.nnz[t]
        crow = torch.empty(cone.row_counts[t] + 1, dtype=torch.int32, device=DEV)
        col = torch.empty(nnz, dtype=torch.int32, device=DEV)
        val = torch.empty(nnz, dtype=torch.float32, device=DEV)
        _hip.check(lib.fly_plan_matrix(plan.handle, t, crow.data_ptr(), col.data_ptr(), val.data_ptr(), st),
                   "fly_plan_matrix")
        assert torch.equal(crow.long(), op.crow) and torch.equal(col.long(), op.pre)
        assert torch.equal(val, w[op.edges])


# ---- the literal recurrence in float64 ---------------------------------------------------------------------------

@pytest.mark.parametrize("h_max", [10.0, None])
def test_literal_recurrence_in_float64(h_max):
    """ConnectomeRNN.forward runs in u's dtype (brain.py:215-223); the reference's tests run it in float64.  The
    float32 weights, alphas and bias widen exactly and every sum and update is float64.  With log_gain = 0 and
    alpha_logit = 0 the float32 transforms (exp, sigmoid) are exact on any implementation, so the device must match
    the oracle's float64 recurrence to 1e-12, on a 3,000-neuron graph and, against the dense brute force, on the
    shuffled control of the reference's test graph (repeated pairs, self-loops); with random parameters it matches
    to float32-parameter round-off (1e-5).  u is left holding u + bias."""
    g = torch.Generator().manual_seed(9)
    for exact in (True, False):
        conn = _medium(8)
        lg, b, al = random_params(conn, 25, gain_sd=0.1, bias_mean=2.0 if h_max is None else 0.1)
        if exact:
            lg, al = np.zeros_like(lg), np.zeros_like(al)
        rnn = _rnn(conn, 4.0, lg, b, al, h_max=h_max)
        ba = brain_arrays(conn, 4.0, lg, b, al, h_max=h_max)          # float32 parameters, as the product's
        ba.w0 = rnn.w0.cpu()
        tol = 1e-12 if exact else 1e-5
        for batch, steps in ((1, 1), (70, 3), (130, 6)):
            u = torch.randn(conn.n_neurons, batch, generator=g, dtype=torch.float64)
            u_dev = u.to(DEV)
            with torch.no_grad():
                h = rnn(u_dev, steps)
            assert h.dtype == torch.float64
            ref = F.literal(ba, u, steps).numpy()
            assert ref.dtype == np.float64
            np.testing.assert_allclose(h.cpu().numpy(), ref, rtol=tol, atol=tol)
            np.testing.assert_array_equal(u_dev.cpu().numpy(),
                                          (u + torch.as_tensor(b).to(torch.float64)[:, None]).numpy())
    conn = tiny_connectome(80, 2000, 4).shuffled(3)
    lg, b, al = random_params(conn, 26, gain_sd=0.3)
    lg, al = np.zeros_like(lg), np.zeros_like(al)
    rnn = _rnn(conn, 3.0, lg, b, al, h_max=h_max)
    W = brute.dense_matrix(conn.n_neurons, conn.pre.numpy(), conn.post.numpy(),
                           (rnn.sign * rnn.w0).cpu().numpy().astype(np.float64))
    alpha = np.full(conn.n_neurons, 0.5)
    u = torch.randn(conn.n_neurons, 33, generator=g, dtype=torch.float64)
    with torch.no_grad():
        h = rnn(u.clone().to(DEV), 5)
    dense = brute.dense_recurrence(W, np.asarray(b, dtype=np.float32).astype(np.float64), alpha, u.numpy(), 5,
                                   h_max=h_max)
    np.testing.assert_allclose(h.cpu().numpy(), dense, rtol=1e-12, atol=1e-12)


# ---- the literal recurrence in float16 ---------------------------------------------------------------------------

@pytest.mark.parametrize("h_max", [10.0, None])
def test_literal_recurrence_in_float16(h_max, sweep_core):
    """ConnectomeRNN.forward with float16 u runs the reference's float16 path (brain.py:213-223): u += bias rounded to
    float16 in place (bit for bit), weights and alpha rounded to float16, a float16 state.  Against the float64
    recurrence over those float16 operands (oracle.forward.literal_f16_operands, the exact function of the path's
    inputs), which the device follows up to its float16 roundings of the state: within 4e-3 of the largest |h| (six
    roundings of 2^-11 of the state and of the sum per step bound it by 6e-3); and against the float32 forward
    within 1e-2 of the largest |h| (the operands' own float16 rounding on top)."""
    conn = _medium(8)
    lg, b, al = random_params(conn, 28, gain_sd=0.1, bias_mean=2.0 if h_max is None else 0.1)
    rnn = _rnn(conn, 4.0, lg, b, al, h_max=h_max)
    ba = brain_arrays(conn, 4.0, lg, b, al, h_max=h_max)               # float32 parameters, as the product's
    ba.w0 = rnn.w0.cpu()
    mat, alpha = F.literal_f16_operands(ba)
    g = torch.Generator().manual_seed(13)
    for batch, steps in ((1, 1), (70, 3), (130, 6)):
        u = torch.randn(conn.n_neurons, batch, generator=g)
        u16 = u.half().to(DEV)
        drive16 = (u.half().float() + torch.as_tensor(b).half().float()[:, None]).half()   # u.add_(bias.half())
        with torch.no_grad():
            h16 = rnn(u16, steps)
            h32 = rnn(u.clone().to(DEV), steps)
        assert h16.dtype == torch.float16
        assert torch.equal(u16.cpu(), drive16), "u + bias in float16, in place"
        h = torch.zeros(conn.n_neurons, batch, dtype=torch.float64)
        for _ in range(steps):
            h = F.literal_step(ba, mat, alpha, h, drive16.double())
        ref = h.numpy()
        scale = max(np.abs(ref).max(), 1e-3)
        err = np.abs(h16.double().cpu().numpy() - ref).max()
        d32 = np.abs(h16.double().cpu().numpy() - h32.double().cpu().numpy()).max()
        print(f"float16 literal {sweep_core} h_max={h_max} B={batch} T={steps}: max |h16 - exact| {err:.2e}, "
              f"|h16 - h32| {d32:.2e} of max |h| {scale:.2e}", flush=True)
        assert err < 4e-3 * scale and d32 < 1e-2 * scale, (batch, steps, err, d32, scale)


# ---- forward_io in float64 ---------------------------------------------------------------------------------------

@pytest.mark.parametrize("h_max", [10.0, None])
def test_forward_io_in_float64(h_max, sweep_core):
    """forward_io with float64 u_in (brain.py:295-329 in u_in's dtype): the float32 cache widens, the state and
    every sum and update are float64, and the outputs come back float64.  With log_gain, bias and alpha_logit zero
    the cache is exact (resting trajectory 0, weights sign * w0, alpha 1/2), so the device matches the float64
    literal recurrence's outputs to 1e-12; with random parameters it matches the oracle's float64 cone over a
    float32 cache within that cache's round-off (1e-5), and the float32 path within float32 round-off."""
    g = torch.Generator().manual_seed(12)
    conn = _medium(8)
    in_idx, out_idx = conn.nodes("afferent"), conn.nodes("efferent")
    ind, outd = in_idx.to(DEV), out_idx.to(DEV)
    for exact in (True, False):
        lg, b, al = random_params(conn, 27, gain_sd=0.1, bias_mean=2.0 if h_max is None else 0.1)
        if exact:
            lg, b, al = np.zeros_like(lg), np.zeros_like(b), np.zeros_like(al)
        rnn = _rnn(conn, 4.0, lg, b, al, h_max=h_max)
        ba = brain_arrays(conn, 4.0, lg, b, al, h_max=h_max)          # float32 parameters, as the product's
        ba.w0 = rnn.w0.cpu()
        for batch, steps in ((1, 1), (70, 3), (130, 6)):
            print(f"float64 forward_io: exact={exact} h_max={h_max} batch={batch} steps={steps}", flush=True)
            u_in = torch.randn(len(in_idx), batch, generator=g, dtype=torch.float64)
            with torch.no_grad():
                out = rnn.forward_io(u_in.to(DEV), ind, outd, steps)
                out32 = rnn.forward_io(u_in.float().to(DEV), ind, outd, steps)
            assert out.dtype == torch.float64 and out.shape == (len(out_idx), batch)
            got = out.cpu().numpy()
            if exact:
                u = torch.zeros(conn.n_neurons, batch, dtype=torch.float64).index_add(0, in_idx, u_in)
                ref = F.literal(ba, u, steps)[out_idx].numpy()
                tol = 1e-12
            else:
                cone = _cone(conn, in_idx, out_idx, steps)
                prep = F.prepare_f32(ba, cone, torch.float64, weights_dtype=torch.float32)
                ref = F.run_f32(prep, steps, u_in).numpy()
                tol = 1e-5
            assert ref.dtype == np.float64
            scale = max(np.abs(ref).max(), 1.0)
            np.testing.assert_allclose(got, ref, rtol=tol, atol=tol * scale)
            np.testing.assert_allclose(out32.cpu().numpy(), got, rtol=2e-5, atol=2e-5 * scale)
