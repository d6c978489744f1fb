"""GPU parity: the HIP evaluator (through the C ABI) against the CPU oracle on the same seeded inputs.

Integer work (light cones, sub-matrices, index tables) must be bit-exact; float32 paths within float32
round-off of the fp64 oracle; the float16 deviation path within the reference's own float16 tolerance and,
for the full model, within 1e-3 max-abs of the float32 path with >= 99.9% policy-argmax agreement."""

from __future__ import annotations

import json
import os
import warnings

import numpy as np
import pytest
import torch

from helpers import REPO, brain_arrays, random_params, tiny_connectome

from oracle import lightcone as L, forward as F

warnings.filterwarnings("ignore", message="Sparse CSR tensor support is in beta")
pytestmark = pytest.mark.gpu

DEV = "cuda:0"
GOLDEN = os.path.join(REPO, "tests", "golden", "fullscale_cone.json")


def product_rnn(conn, scale, lg, b, al, h_max=10.0):
    from chessfly.brain import ConnectomeRNN
    rnn = ConnectomeRNN(conn, global_scale=scale, h_max=h_max)
    with torch.no_grad():
        rnn.log_gain.copy_(torch.as_tensor(lg))
        rnn.bias.copy_(torch.as_tensor(b))
        rnn.alpha_logit.copy_(torch.as_tensor(al))
    return rnn.to(DEV)


def oracle_cone(conn, in_idx, out_idx, steps):
    return L.light_cone(conn.n_neurons, conn.pre.numpy(), conn.post.numpy(), np.asarray(in_idx), np.asarray(out_idx),
                        steps)


def assert_cone_equal(cone, ref):
    """Every LightCone attribute of the device cone equals the oracle's, element for element."""
    cpu = lambda t: t.detach().cpu().numpy()
    assert cone.steps == ref.steps
    for t in range(ref.steps + 1):
        np.testing.assert_array_equal(cpu(cone.rows[t]), ref.rows[t])
    for t in range(1, ref.steps + 1):
        if ref.ops[t] is None:
            assert cone.ops[t] is None
        else:
            op, rop = cone.ops[t], ref.ops[t]
            assert op.shape == rop.shape
            for name in ("edges", "post", "pre", "crow"):
                np.testing.assert_array_equal(cpu(getattr(op, name)), getattr(rop, name), err_msg=f"{name} t={t}")
        for name in ("keep_next", "keep_prev", "prev_row", "u_pos", "u_src"):
            np.testing.assert_array_equal(cpu(getattr(cone, name)[t]), getattr(ref, name)[t], err_msg=f"{name} t={t}")
        np.testing.assert_array_equal(cpu(cone.carried[t]).reshape(-1), ref.carried[t])
    np.testing.assert_array_equal(cpu(cone.out_pos), ref.out_pos)
    np.testing.assert_array_equal(cpu(cone.out_src), ref.out_src)
    assert cone.edge_visits == ref.edge_visits


TINY = [(120, 700, 3, np.arange(0, 9), np.arange(100, 120)),
        (30, 200, 0, np.arange(0, 5), np.arange(25, 30)),
        (60, 600, 1, np.array([3, 7, 11, 40]), np.array([0, 7, 59]))]


@pytest.mark.parametrize("n,e,seed,in_idx,out_idx", TINY)
@pytest.mark.parametrize("steps", [0, 1, 2, 4, 6])
def test_light_cone_bit_exact_tiny(n, e, seed, in_idx, out_idx, steps):
    conn = tiny_connectome(n, e, seed)
    rnn = product_rnn(conn, 3.0, *random_params(conn, 1))
    cone = rnn.light_cone(torch.as_tensor(in_idx, device=DEV), torch.as_tensor(out_idx, device=DEV), steps)
    assert_cone_equal(cone, oracle_cone(conn, in_idx, out_idx, steps))


def test_light_cone_bit_exact_on_shuffled_control_with_repeats():
    conn = tiny_connectome(80, 2000, 4).shuffled(3)
    rnn = product_rnn(conn, 2.0, *random_params(conn, 2))
    in_idx, out_idx = np.arange(0, 10), np.arange(60, 80)
    for steps in (3, 6):
        cone = rnn.light_cone(torch.as_tensor(in_idx, device=DEV), torch.as_tensor(out_idx, device=DEV), steps)
        assert_cone_equal(cone, oracle_cone(conn, in_idx, out_idx, steps))


@pytest.mark.parametrize("steps", [1, 3, 6])
def test_unpruned_cone_bit_exact_and_same_function(steps):
    """Pruning off (every neuron, every step) builds the trivial cone bit-exactly and computes the same
    outputs as the pruned cone, in both state modes."""
    conn = tiny_connectome(120, 700, seed=3)
    lg, b, al = random_params(conn, 4)
    rnn = product_rnn(conn, 3.0, lg, b, al)
    in_idx, out_idx = np.arange(0, 9), np.arange(100, 120)
    ind, outd = torch.as_tensor(in_idx, device=DEV), torch.as_tensor(out_idx, device=DEV)
    u = torch.randn(9, 33, generator=torch.Generator().manual_seed(steps)).to(DEV)
    with torch.no_grad():
        outs = {}
        for prune in (True, False):
            cone = rnn.light_cone(ind, outd, steps, prune=prune)
            ref = L.light_cone(conn.n_neurons, conn.pre.numpy(), conn.post.numpy(), in_idx, out_idx, steps, prune=prune)
            assert_cone_equal(cone, ref)
            outs[prune] = (rnn.forward_io(u, ind, outd, steps), rnn.forward_io(u.half(), ind, outd, steps))
    torch.testing.assert_close(outs[True][0], outs[False][0], rtol=2e-5, atol=2e-5)
    torch.testing.assert_close(outs[True][1], outs[False][1], rtol=5e-3, atol=5e-3)


def _medium(seed=0):
    from chessfly.synthetic import GraphSpec, synthetic_connectome
    spec = GraphSpec(n=3000, edges=120_000, n_sensory=300, n_output=80, seed=seed)
    return synthetic_connectome(spec)


@pytest.mark.parametrize("batch", [1, 5, 64, 200])
def test_literal_recurrence_matches_oracle(batch):
    conn = _medium()
    lg, b, al = random_params(conn, 5, gain_sd=0.1)
    rnn = product_rnn(conn, 4.0, lg, b, al)
    ba = brain_arrays(conn, 4.0, lg, b, al, dtype=torch.float64)
    g = torch.Generator().manual_seed(batch)
    u = torch.randn(conn.n_neurons, batch, generator=g) * 0.5
    for steps in (0, 1, 3, 6):
        u_dev = u.to(DEV)
        with torch.no_grad():
            h = rnn(u_dev, steps)
        torch.cuda.synchronize()
        ref = F.literal(ba, u.double(), steps)
        np.testing.assert_allclose(h.cpu().numpy(), ref.numpy(), rtol=2e-5, atol=2e-5)
        # the reference's inference path leaves u + bias in u
        np.testing.assert_allclose(u_dev.cpu().numpy(), (u + torch.as_tensor(b)[:, None]).numpy(), rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("batch", [1, 7, 64, 130])
@pytest.mark.parametrize("steps", [1, 2, 4, 6])
def test_cone_forward_f32_matches_oracle_and_literal(batch, steps):
    conn = _medium(1)
    lg, b, al = random_params(conn, 6, gain_sd=0.1)
    rnn = product_rnn(conn, 4.0, lg, b, al)
    ba = brain_arrays(conn, 4.0, lg, b, al, dtype=torch.float64)
    in_idx, out_idx = conn.nodes("afferent"), conn.nodes("efferent")
    u_in = torch.randn(len(in_idx), batch, generator=torch.Generator().manual_seed(steps)) * 0.5
    with torch.no_grad():
        out = rnn.forward_io(u_in.to(DEV), in_idx.to(DEV), out_idx.to(DEV), steps)
        u = torch.zeros(conn.n_neurons, batch, device=DEV).index_add_(0, in_idx.to(DEV), u_in.to(DEV))
        lit = rnn(u, steps)[out_idx.to(DEV)]
    cone = oracle_cone(conn, in_idx, out_idx, steps)
    ref = F.cone_f32(ba, cone, u_in.double(), steps)
    assert out.dtype == torch.float32 and out.shape == (len(out_idx), batch)
    np.testing.assert_allclose(out.cpu().numpy(), ref.numpy(), rtol=2e-5, atol=2e-5)
    np.testing.assert_allclose(out.cpu().numpy(), lit.cpu().numpy(), rtol=2e-5, atol=2e-5)


def test_half_precision_inference_matches_float32():
    """tests/test_core.py:491-511 on the device: a small signal on a large resting state, rows clamped below
    zero and above h_max; the float16 deviation path must stay within 0.02 * signal + 1e-4 of float32."""
    conn = tiny_connectome(400, 9000, seed=5)
    g = torch.Generator().manual_seed(0)
    lg = (torch.randn(conn.n_edges, generator=g) * 0.8).numpy()
    b = (0.6 + torch.randn(conn.n_neurons, generator=g) * 0.7).numpy()
    b[::17] += 12.0
    al = torch.randn(conn.n_neurons, generator=g).numpy()
    rnn = product_rnn(conn, 2.0, lg, b, al)
    in_idx, out_idx = torch.arange(0, 40, device=DEV), torch.arange(300, 400, device=DEV)
    u = (torch.randn(40, 64, generator=g) * 0.05).to(DEV)
    ba = brain_arrays(conn, 2.0, lg, b, al, dtype=torch.float64)
    with torch.no_grad():
        for steps in (1, 3, 6):
            ref = rnn.forward_io(u, in_idx, out_idx, steps)
            half = rnn.forward_io(u.half(), in_idx, out_idx, steps)
            assert half.dtype == torch.float32
            signal = (ref - ref.mean(1, keepdim=True)).abs().mean()
            assert float((half - ref).abs().max()) < 0.02 * float(signal) + 1e-4
            # and at least as close to the exact function as the reference's float16 emulation
            cone = oracle_cone(conn, in_idx.cpu(), out_idx.cpu(), steps)
            exact = F.cone_f32(ba, cone, u.cpu().double(), steps).numpy()
            ours = np.abs(half.cpu().numpy() - exact).max()
            emulated = np.abs(F.cone_half(brain_arrays(conn, 2.0, lg, b, al), cone, u.cpu(), steps).numpy() - exact).max()
            assert ours <= emulated + 1e-6, (steps, ours, emulated)


@pytest.mark.parametrize("batch", [1, 3, 64, 100])
def test_deviation_path_matches_exact_function(batch):
    conn = _medium(2)
    lg, b, al = random_params(conn, 8, gain_sd=0.1)
    rnn = product_rnn(conn, 4.0, lg, b, al)
    ba = brain_arrays(conn, 4.0, lg, b, al, dtype=torch.float64)
    in_idx, out_idx = conn.nodes("afferent"), conn.nodes("efferent")
    u_in = torch.randn(len(in_idx), batch, generator=torch.Generator().manual_seed(batch))
    steps = 6
    with torch.no_grad():
        out = rnn.forward_io(u_in.half().to(DEV), in_idx.to(DEV), out_idx.to(DEV), steps)
    cone = oracle_cone(conn, in_idx, out_idx, steps)
    exact = F.cone_f32(ba, cone, u_in.half().double(), steps).numpy()
    err = np.abs(out.cpu().numpy() - exact).max()
    dev_scale = np.abs(exact - F.cone_f32(ba, cone, torch.zeros_like(u_in).double(), steps).numpy()).max()
    assert err < 2e-3 * max(dev_scale, 1e-3), (err, dev_scale)


STEP_SHAPES = [{"groups": 4}, {"groups": 2}, {"groups": 1}, {"groups": 1, "unroll": 16}, {"groups": 1, "unroll": 32},
               {"rows_mode": 1}, {"rows_mode": 1, "groups": 4}, {"rows_mode": 1, "unroll": 8}, {"rows_mode": -1},
               {"rows_mode": 1, "rows_vec": 8}, {"rows_mode": 1, "rows_vec": 16}, {"rows_mode": 1, "rows_vec": 16, "unroll": 8},
               {"vec": 4}, {"vec": 2}, {"vec": 1}, {"nt_store": 1}]


@pytest.fixture
def step_shape(request):
    from chessfly import _hip
    for key, value in request.param.items():
        _hip.set_tuning(key, value)
    yield request.param
    for key in request.param:
        _hip.set_tuning(key, 0)


@pytest.mark.parametrize("step_shape", STEP_SHAPES, indirect=True, ids=lambda p: "-".join(f"{k}{v}" for k, v in p.items()))
def test_every_step_kernel_shape_matches_the_oracle(step_shape):
    """Every lane-group, row-slot, unroll and lane-width variant of the state step (selected with
    fly_set_tuning) computes the same function: the fp16 deviation path within its tolerance of the exact
    function and the float32 light cone within float32 round-off, at a batch that ends inside a chunk."""
    conn = _medium(2)
    lg, b, al = random_params(conn, 8, gain_sd=0.1)
    rnn = product_rnn(conn, 4.0, lg, b, al)
    ba = brain_arrays(conn, 4.0, lg, b, al, dtype=torch.float64)
    in_idx, out_idx = conn.nodes("afferent"), conn.nodes("efferent")
    batch, steps = 100, 6
    u_in = torch.randn(len(in_idx), batch, generator=torch.Generator().manual_seed(3))
    cone = oracle_cone(conn, in_idx, out_idx, steps)
    with torch.no_grad():
        half = rnn.forward_io(u_in.half().to(DEV), in_idx.to(DEV), out_idx.to(DEV), steps)
        full = rnn.forward_io(u_in.to(DEV), in_idx.to(DEV), out_idx.to(DEV), steps)
    exact = F.cone_f32(ba, cone, u_in.half().double(), steps).numpy()
    dev_scale = np.abs(exact - F.cone_f32(ba, cone, torch.zeros_like(u_in).double(), steps).numpy()).max()
    err = np.abs(half.cpu().numpy() - exact).max()
    assert err < 2e-3 * max(dev_scale, 1e-3), (err, dev_scale)
    np.testing.assert_allclose(full.cpu().numpy(), F.cone_f32(ba, cone, u_in.double(), steps).numpy(),
                               rtol=2e-5, atol=2e-5)


def _dense_plan(lib, _hip, n_in, k, ld, n_out, moves, rng, scale_w=0.05):
    """A dense plan over random weights; returns (handle, host copies of the weights)."""
    import ctypes
    from chessfly.encoding import move_squares
    frm, to = move_squares()
    T = lambda a: torch.as_tensor(np.asarray(a, dtype=np.float32))
    P = dict(enc_w=rng.normal(0, scale_w, (n_in, ld)), enc_b=rng.normal(0, scale_w, n_in),
             policy_w=rng.normal(0, 0.1, (moves, n_out)), policy_b=rng.normal(0, 0.1, moves),
             from_w=rng.normal(0, 0.1, (64, n_out)), from_b=rng.normal(0, 0.1, 64),
             to_w=rng.normal(0, 0.1, (64, n_out)), to_b=rng.normal(0, 0.1, 64),
             value_w=rng.normal(0, 0.1, (3, n_out)), value_b=rng.normal(0, 0.1, 3),
             mean=rng.normal(0, 1, n_out), var=rng.uniform(0.01, 2, n_out))
    dev = {key: T(v).to(DEV).contiguous() for key, v in P.items()}
    mf = torch.as_tensor(frm[:moves].astype(np.int32), device=DEV)
    mt = torch.as_tensor(to[:moves].astype(np.int32), device=DEV)
    desc = _hip.HeadDesc(n_out, moves, dev["mean"].data_ptr(), dev["var"].data_ptr(), 1e-8, 8.0,
                         dev["policy_w"].data_ptr(), dev["policy_b"].data_ptr(), dev["from_w"].data_ptr(),
                         dev["from_b"].data_ptr(), dev["to_w"].data_ptr(), dev["to_b"].data_ptr(),
                         dev["value_w"].data_ptr(), dev["value_b"].data_ptr(), mf.data_ptr(), mt.data_ptr())
    h = ctypes.c_void_p()
    _hip.check(lib.fly_dense_create(ctypes.byref(desc), dev["enc_w"].data_ptr(), ld, k, dev["enc_b"].data_ptr(), n_in,
                                    _hip.stream(torch.device(DEV)), ctypes.byref(h)), "fly_dense_create")
    return _hip.Handle(h, "fly_dense_destroy"), {key: T(v) for key, v in P.items()}, frm[:moves], to[:moves]


@pytest.fixture
def gemm_tile(request):
    from chessfly import _hip
    _hip.set_tuning("gemm_tile", request.param)
    yield request.param
    _hip.set_tuning("gemm_tile", 0)


@pytest.mark.parametrize("gemm_tile", [0, 1, 2, 3, 24, 25, 32, 34, 35, 45], indirect=True)
@pytest.mark.parametrize("batch,n_in,k,ld,n_out,moves", [(5, 70, 30, 33, 40, 100), (130, 300, 838, 967, 150, 4168),
                                                          (1, 17, 838, 967, 2333, 4168)])
def test_encoder_and_head_gemms_match_fp64(batch, n_in, k, ld, n_out, moves, gemm_tile):
    """The split-fp16 matrix-core GEMMs hold float32 accuracy: encoder and head against fp64, for every workgroup
    tile shape (0: the automatic choice)."""
    from chessfly import _hip
    from oracle.forward import HeadArrays
    lib = _hip.load()
    rng = np.random.default_rng(batch)
    dense, P, frm, to = _dense_plan(lib, _hip, n_in, k, ld, n_out, moves, rng)
    x = torch.as_tensor(rng.random((batch, ld)) < 0.1, dtype=torch.float32)
    # Values not representable in fp16 in the first three boards only: their tile runs the product with the boards'
    # low half, the tiles of the later boards (exact in fp16) leave it out.
    x[:3, 0] = 0.37
    x[:3, 1] = 1.0 / 3.0
    ref = ((x[:, :k].double() @ P["enc_w"][:, :k].double().T + P["enc_b"].double()) * 5.0).T
    xd = x.to(DEV)
    ws = _hip.workspace(lib.fly_encoder_workspace(dense.handle, batch), torch.device(DEV))
    for f16 in (0, 1):
        ldu = batch + 3
        u = torch.zeros(n_in, ldu, dtype=torch.float16 if f16 else torch.float32, device=DEV)
        _hip.check(lib.fly_encoder(dense.handle, xd.data_ptr(), 0, ld, batch, 5.0, u.data_ptr(), ldu, f16,
                                   ws.data_ptr(), ws.numel(), _hip.stream(torch.device(DEV))), "fly_encoder")
        got = u[:, :batch].double().cpu()
        tol = ref.abs() * (2 ** -10) + 1e-6 if f16 else ref.abs() * 2e-6 + 2e-6
        assert bool(((got - ref).abs() <= tol).all()), float((got - ref).abs().max())
        assert bool((u[:, batch:] == 0).all())             # the padding columns past the batch stay untouched
    # Half-precision boards (what the search sends) widen exactly: the same bits as their float32 copy.
    xh = x.half().to(DEV)
    u_h, u_f = (torch.zeros(n_in, batch, device=DEV) for _ in range(2))
    for src, is_half, u in ((xh, 1, u_h), (xh.float(), 0, u_f)):
        _hip.check(lib.fly_encoder(dense.handle, src.data_ptr(), is_half, ld, batch, 5.0, u.data_ptr(), batch, 0,
                                   ws.data_ptr(), ws.numel(), _hip.stream(torch.device(DEV))), "fly_encoder")
    assert torch.equal(u_h, u_f)
    r = torch.as_tensor(rng.normal(0, 3, (n_out, batch)), dtype=torch.float32)
    logits = torch.empty(batch, moves, device=DEV)
    wdl = torch.empty(batch, 3, device=DEV)
    ws = _hip.workspace(lib.fly_head_workspace(dense.handle, batch), torch.device(DEV))
    rd = r.to(DEV)
    _hip.check(lib.fly_head(dense.handle, rd.data_ptr(), batch, batch, logits.data_ptr(), wdl.data_ptr(), ws.data_ptr(),
                            ws.numel(), _hip.stream(torch.device(DEV))), "fly_head")
    d = lambda key: P[key].double()
    hp = HeadArrays(None, None, 5.0, 0, d("policy_w"), d("policy_b"), d("from_w"), d("from_b"), d("to_w"), d("to_b"),
                    d("value_w"), d("value_b"), torch.as_tensor(frm), torch.as_tensor(to), d("mean"), d("var"))
    ref_l, ref_w = F.heads(hp, F.norm(hp, r.double().T))
    # float32 accuracy: no worse than torch's own float32 head on the CPU, measured against fp64
    hp32 = HeadArrays(None, None, 5.0, 0, *[P[k_] for k_ in ("policy_w", "policy_b", "from_w", "from_b", "to_w", "to_b",
                                                              "value_w", "value_b")],
                      torch.as_tensor(frm), torch.as_tensor(to), P["mean"], P["var"])
    cpu_l, cpu_w = F.heads(hp32, F.norm(hp32, r.T))
    for got, ref, cpu in ((logits, ref_l, cpu_l), (wdl, ref_w, cpu_w)):
        ours = float((got.cpu().double() - ref).abs().max())
        theirs = float((cpu.double() - ref).abs().max())
        assert ours <= 3 * theirs + 1e-6 * float(ref.abs().max()), (ours, theirs)


# ---- full scale (166,700 neurons, 10.5M synapses) ------------------------------------------------------------

def _record_from_device(cone, in_idx):
    """The golden-record digests of a device cone (same fields as tests/golden/make_golden.py)."""
    from golden.make_golden import digest
    steps = []
    for t in range(cone.steps + 1):
        rec = {"rows": int(cone.row_counts[t]), "rows_sha": digest(cone.rows[t].cpu().numpy())}
        if t >= 1:
            nr = cone.row_counts[t]
            prev = torch.empty(nr, dtype=torch.int32, device=DEV)
            usrc = torch.empty(nr, dtype=torch.int32, device=DEV)
            cone._step_export(t, prev=prev, usrc=usrc)
            rec.update(prev_sha=digest(prev.cpu().numpy()), usrc_sha=digest(usrc.cpu().numpy()),
                       carried=int((prev >= 0).sum()), fed=int((usrc >= 0).sum()))
            if cone.ops[t] is None:
                rec.update(op=False, nnz=0)
            else:
                op = cone.ops[t]
                rec.update(op=True, nnz=int(cone.nnz[t]), crow_sha=digest(op.crow.cpu().numpy()),
                           col_sha=digest(op.pre.cpu().numpy()), edge_sha=digest(op.edges.cpu().numpy()))
        steps.append(rec)
    src = torch.full((cone.n_out,), -1, dtype=torch.long, device=DEV)
    src[cone.out_pos] = cone.out_src
    return {"steps": steps, "edge_visits": int(cone.edge_visits), "out_src_sha": digest(src.cpu().numpy()),
            "out_hit": int(len(cone.out_pos))}


@pytest.mark.parametrize("graph", ["synthetic", "shuffled"])
def test_full_scale_light_cone_bit_exact(graph, full_net):
    with open(GOLDEN) as f:
        gold = json.load(f)["graphs"][graph]
    net, conn = full_net
    if graph == "shuffled":
        from chessfly.brain import ConnectomeRNN
        conn = conn.shuffled(0)
        rnn = ConnectomeRNN(conn).to(DEV)
    else:
        rnn = net.brain
    in_idx, out_idx = conn.nodes("afferent").to(DEV), conn.nodes("efferent").to(DEV)
    for steps in ("6", "4"):
        cone = rnn.light_cone(in_idx, out_idx, int(steps))
        assert _record_from_device(cone, in_idx) == gold["cones"][steps], (graph, steps)


def _oracle_full(conn):
    from chessfly.synthetic import synthetic_maps, synthetic_params
    from chessfly.encoding import N_BASE, move_squares
    from helpers import head_arrays
    p = synthetic_params(conn, seed=0)
    ba = brain_arrays(conn, p.global_scale, p.log_gain, p.bias, p.alpha_logit)
    in_idx, out_idx = conn.nodes("afferent"), conn.nodes("efferent")
    frm, to = move_squares()
    hp = head_arrays(synthetic_maps(len(in_idx), len(out_idx), 0), 5.0, N_BASE, frm, to, len(out_idx))
    cone = oracle_cone(conn, in_idx, out_idx, 6)
    return ba, hp, cone


def test_full_scale_model_matches_oracle(full_net):
    """FlyChessNet.forward at full scale, float32 and float16-deviation paths, against the oracle's float32
    forward on 24 boards: policy logits and WDL within 1e-3 max-abs, argmax equal."""
    from chessfly.synthetic import synthetic_boards
    net, conn = full_net
    ba, hp, cone = _oracle_full(conn)
    x = torch.as_tensor(synthetic_boards(24, seed=11))
    ref_logits, ref_wdl = F.model_forward(ba, hp, cone, x, "f32")
    for dtype in (torch.float32, torch.float16):
        net.infer_dtype = dtype
        with torch.no_grad():
            logits, wdl = net(x.to(DEV))
        torch.cuda.synchronize()
        dl = float((logits.cpu() - ref_logits).abs().max())
        dw = float((wdl.cpu() - ref_wdl).abs().max())
        print(f"{dtype}: max |logit diff| {dl:.3e}  max |wdl diff| {dw:.3e}", flush=True)
        assert dl < 1e-3 and dw < 1e-3, (dtype, dl, dw)
        assert torch.equal(logits.cpu().argmax(1), ref_logits.argmax(1))
    net.infer_dtype = torch.float16


def test_full_scale_outputs_do_not_depend_on_the_batch(full_net):
    """A board's logits do not depend on the batch around it: the first boards of batches of 1, 65, 2100, 4096 and
    8192 match the 24-board forward, float32 within float32 round-off of the summation order and float16
    deviation within its tolerance; at every size the float16 deviation path agrees with float32 within 1e-3 and
    on >= 99.9% of the argmaxes.  Batches whose state would pass 2 GiB (float32 from about 3,200 boards, float16
    from about 6,400) run as column blocks."""
    from chessfly.synthetic import synthetic_boards
    net, _ = full_net
    x = torch.as_tensor(synthetic_boards(8192, seed=21)).to(DEV)
    ref = {}
    for dtype in (torch.float32, torch.float16):
        net.infer_dtype = dtype
        with torch.no_grad():
            ref[dtype] = net(x[:24])
    try:
        for batch in (1, 65, 2100, 4096, 8192):
            out = {}
            for dtype in (torch.float32, torch.float16):
                net.infer_dtype = dtype
                with torch.no_grad():
                    out[dtype] = net(x[:batch])
                k = min(batch, 24)
                tol = 5e-5 if dtype == torch.float32 else 1e-3
                dl = float((out[dtype][0][:k] - ref[dtype][0][:k]).abs().max())
                dw = float((out[dtype][1][:k] - ref[dtype][1][:k]).abs().max())
                print(f"B={batch} {dtype}: first {k} boards vs B=24: {dl:.2e} / {dw:.2e}", flush=True)
                assert dl < tol and dw < tol, (batch, dtype, dl, dw)
            (l32, w32), (l16, w16) = out[torch.float32], out[torch.float16]
            assert float((l16 - l32).abs().max()) < 1e-3 and float((w16 - w32).abs().max()) < 1e-3
            assert float((l16.argmax(1) == l32.argmax(1)).float().mean()) >= 0.999
    finally:
        net.infer_dtype = torch.float16


def test_full_scale_blocked_columns_match_unblocked(full_net):
    """forward_io and the literal recurrence over more columns than fit one 2 GiB float32 state (run as column
    blocks) give the same columns as a call on those columns alone."""
    net, _ = full_net
    rnn = net.brain
    g = torch.Generator().manual_seed(5)
    with torch.no_grad():
        u_in = (torch.randn(len(net.in_idx), 4100, generator=g) * 0.5).to(DEV)
        big = rnn.forward_io(u_in, net.in_idx, net.out_idx, 6)
        for cols in (slice(0, 24), slice(4076, 4100)):
            small = rnn.forward_io(u_in[:, cols].contiguous(), net.in_idx, net.out_idx, 6)
            torch.testing.assert_close(big[:, cols], small, rtol=0, atol=2e-5)
        u = (torch.randn(rnn.n, 3300, generator=g) * 0.5).to(DEV)
        head, tail = u[:, :24].clone(), u[:, -24:].clone()
        h = rnn(u, 4)
        torch.testing.assert_close(h[:, :24], rnn(head, 4), rtol=0, atol=2e-5)
        torch.testing.assert_close(h[:, -24:], rnn(tail, 4), rtol=0, atol=2e-5)


def test_full_scale_swept_steps_match_the_grouped_kernel(full_net):
    """The long-row steps (166,539-166,700 and 77,286 rows of ~63 non-zeros over 166K sources) run as a banded sweep
    of the sources (k_state_step_swept: 4 bands, or 3 from the sweep_bands tuning; one or two rows per pass; rows in
    index order or longest first; passes of 6 or 3 slots, with or without the next rounds' gathers in flight); with
    the sweep off (tuning swept=-1) they run on the grouped kernel.  Same sums
    in another order: float16 deviation logits agree within 5e-4 and float32 within 2e-5, with the argmax on
    >= 99.9% of 1120 boards."""
    from chessfly import _hip
    from chessfly.synthetic import synthetic_boards
    net, _ = full_net
    x = torch.as_tensor(synthetic_boards(1120, seed=23), device=DEV)

    def run():
        with torch.no_grad():
            net.brain.bias.add_(0.0)            # a new parameter version: the next forward builds a new plan
            out = net(x)
        torch.cuda.synchronize()
        return out

    try:
        for dtype, tol in ((torch.float16, 5e-4), (torch.float32, 2e-5)):
            net.infer_dtype = dtype
            _hip.set_tuning("swept", -1)
            grouped = run()
            _hip.set_tuning("swept", 0)
            variants = {}
            for label, key, value in (("default", "sweep_bands", 0), ("3 bands", "sweep_bands", 3),
                                      ("index order", "sweep_order", -1), ("two rows per pass", "sweep_paired", 1),
                                      ("one row per pass", "sweep_paired", -1), ("3-slot passes", "sweep_slots", 3),
                                      ("pipelined 6 slots", "sweep_pipe", 1), ("never pipelined", "sweep_pipe", -1)):
                _hip.set_tuning(key, value)
                variants[label] = run()
                _hip.set_tuning(key, 0)
            for label, (lg, wd) in variants.items():
                dl = float((lg - grouped[0]).abs().max())
                dw = float((wd - grouped[1]).abs().max())
                agree = float((lg.argmax(1) == grouped[0].argmax(1)).float().mean())
                print(f"{dtype} swept ({label}) vs grouped: logits {dl:.3e}, wdl {dw:.3e}, argmax {agree:.4%}",
                      flush=True)
                assert dl < tol and dw < tol and agree >= 0.999, (dtype, label, dl, dw, agree)
            assert not torch.equal(variants["default"][0], grouped[0])     # the sweep did run
    finally:
        for key in ("swept", "sweep_bands", "sweep_order", "sweep_paired", "sweep_slots", "sweep_pipe"):
            _hip.set_tuning(key, 0)
        net.infer_dtype = torch.float16


def _unit_rounds_numpy(vals, r, paired):
    """Rounds of swept units summed over the bands, as the plan's searches count them.  vals (..., bands, U): band
    counts at the unit's positions; r (...): positions holding rows.  A unit is a slot of 8 positions (the longest
    share of its rows, a slot of r <= 4 rows spreading each over 2, 4 or 8 groups) or, paired, two slots walked as
    one pass (the largest sum of a lane group's two rows); padded to 4 rounds per band."""
    U = vals.shape[-1]
    live = np.arange(U) < r[..., None, None]
    v = np.where(live, vals, 0)
    if paired:
        mx = (v[..., :8] + v[..., 8:]).max(axis=-1)
    else:
        lf = np.where(r >= 5, 0, np.where(r >= 3, 1, np.where(r == 2, 2, 3)))[..., None, None]
        mx = ((v + (1 << lf) - 1) >> lf).max(axis=-1)
    return ((mx + 3) & ~3).sum(axis=-1)


def _balance_numpy(order, cnt, per, groups, steps, paired=False):
    """The plan's balance search restated for the given groups of 16 segments: cost = per band, 16 x the largest of
    the group's wave totals plus their sum; at each step each of 256 threads (xorshift32 per group and thread) draws
    two positions of the group, scores the change a swap of their rows would make (the other waves' largest total
    from the band's three largest), and the lowest score (ties: lowest thread) is made if it adds no cost."""
    bands = cnt.shape[1]
    nr = len(order)      # positions of the order
    W, L = 16, 256
    U = 16 if paired else 8
    order = order.copy()
    G = len(groups)
    starts = np.asarray(groups) * W * per
    M = np.minimum(W * per, nr - starts)
    pos = np.arange(W * per)
    rows = np.where(pos[None, :] < M[:, None], order[np.minimum(starts[:, None] + pos[None, :], nr - 1)], -1)
    c = np.where(rows[:, None, :] >= 0, cnt[np.maximum(rows, 0)].transpose(0, 2, 1), 0)   # (G, bands, W * per)
    rows_of = np.clip(M[:, None] - np.arange(W)[None, :] * per, 0, per)
    gix = np.arange(G)[:, None, None, None]
    bix = np.arange(bands)[None, None, :, None]
    def rounds(w, j, x, y):   # (G, X) -> (G, X, bands) per band rounds of wave w's unit j with rows x, y swapped
        r = np.clip(np.take_along_axis(rows_of, w, 1) - U * j, 0, U)
        p = w[..., None] * per + U * j[..., None] + np.arange(U)
        src = np.where(p == x[..., None], y[..., None], np.where(p == y[..., None], x[..., None], p))
        vals = c[gix, bix, np.minimum(src, W * per - 1)[:, :, None, :]]                   # (G, X, bands, U)
        out = np.stack([_unit_rounds_numpy(vals[:, :, q:q + 1, :], r, paired) for q in range(bands)], axis=-1)
        return np.where(r[..., None] > 0, out, 0)
    nu = 64 // U
    ww, jj = np.meshgrid(np.arange(W), np.arange(nu), indexing="ij")
    ww = np.tile(ww.reshape(1, -1), (G, 1)); jj = np.tile(jj.reshape(1, -1), (G, 1))
    sr = rounds(ww, jj, np.full_like(ww, -1), np.full_like(ww, -1)).reshape(G, W, nu, bands)
    tot = sr.sum(axis=2)
    def top3():
        o = np.lexsort((np.broadcast_to(np.arange(W)[None, :, None], tot.shape), -tot), axis=1)[:, :3, :]
        return np.take_along_axis(tot, o, 1), o
    tv, ti = top3()
    low = np.uint64(0xFFFFFFFF)
    gg = np.asarray(groups, dtype=np.uint64)[:, None]
    tt = np.arange(L, dtype=np.uint64)[None, :]
    state = ((np.uint64(2463534242) ^ ((gg * np.uint64(2654435761)) & low) ^ (((tt + np.uint64(1)) * np.uint64(2246822507)) & low))
             | np.uint64(1)).astype(np.uint32)
    def nxt():
        nonlocal state
        state = state ^ (state << np.uint32(13))
        state = state ^ (state >> np.uint32(17))
        state = state ^ (state << np.uint32(5))
        return state
    ag = np.arange(G)
    for _ in range(steps):
        p1 = (nxt() % M[:, None].astype(np.uint32)).astype(np.int64)
        p2 = (nxt() % M[:, None].astype(np.uint32)).astype(np.int64)
        w1, j1, w2, j2 = p1 // per, (p1 % per) // U, p2 // per, (p2 % per) // U
        same = (w1 == w2) & (j1 == j2)
        valid = ~same | (paired & (((p1 % per) & 7) != ((p2 % per) & 7)))
        a1 = rounds(w1, j1, p1, p2)
        a2 = np.where(same[..., None], a1, rounds(w2, j2, p1, p2))
        s1, s2, s12 = sr[ag[:, None], w1, j1], sr[ag[:, None], w2, j2], sr[ag[:, None], w1, j2]
        T1, T2 = tot[ag[:, None], w1], tot[ag[:, None], w2]
        sw = ((w1 == w2) & ~same)[..., None]
        t1 = np.where(same[..., None], T1 - s1 + a1, np.where(sw, T1 - s1 - s12 + a1 + a2, T1 - s1 + a1))
        t2 = np.where((w1 == w2)[..., None], t1, T2 - s2 + a2)
        ok = (ti[:, None, :, :] != w1[:, :, None, None]) & (ti[:, None, :, :] != w2[:, :, None, None])
        first = np.argmax(ok, axis=2)
        other = np.maximum(np.take_along_axis(np.broadcast_to(tv[:, None], ok.shape), first[:, :, None, :], 2)[:, :, 0, :], 0)
        newmax = np.maximum(other, np.maximum(t1, t2))
        dsum = np.where((w1 == w2)[..., None], t1 - T1, (t1 - T1) + (t2 - T2))
        d = (W * (newmax - tv[:, None, 0, :]) + dsum).sum(axis=2)
        d = np.where(valid, d, 1 << 20)
        win = np.argmin(((d + (1 << 20)) << 8) | np.arange(L)[None, :], axis=1)
        for g in np.nonzero(d[ag, win] <= 0)[0]:
            x = win[g]
            q1, q2 = p1[g, x], p2[g, x]
            rows[g, [q1, q2]] = rows[g, [q2, q1]]
            c[g][:, [q1, q2]] = c[g][:, [q2, q1]]
            v1, v2, k1, k2 = w1[g, x], w2[g, x], j1[g, x], j2[g, x]
            if same[g, x]:
                tot[g, v1] += a1[g, x] - sr[g, v1, k1]
            elif v1 == v2:
                tot[g, v1] += a1[g, x] - sr[g, v1, k1] + a2[g, x] - sr[g, v1, k2]
            else:
                tot[g, v1] += a1[g, x] - sr[g, v1, k1]
                tot[g, v2] += a2[g, x] - sr[g, v2, k2]
            sr[g, v1, k1] = a1[g, x]
            sr[g, v2, k2] = a2[g, x]
        tv, ti = top3()
    for g in range(G):
        order[starts[g]:starts[g] + M[g]] = rows[g, :M[g]]
    return order


def _deal_numpy(items, vlen, caps):
    """Items (longest first) dealt to waves of the given capacities: cut into units of 8 consecutive items, as many
    as whole units fit the waves; each unit to the wave with the least work that has room for a whole unit, then the
    items left each to the wave with the least work that has a free position (ties: the lower wave)."""
    import heapq
    units = sum(c // 8 for c in caps)
    bins = [[] for _ in caps]
    work = [0] * len(caps)
    heap = [(0, w) for w in range(len(caps)) if caps[w] >= 8]
    heapq.heapify(heap)
    for u in range(units):
        wk, w = heapq.heappop(heap)
        unit = items[8 * u: 8 * u + 8]
        bins[w].extend(unit)
        work[w] = wk + int(vlen[unit].sum())
        if len(bins[w]) + 8 <= caps[w]:
            heapq.heappush(heap, (work[w], w))
    heap = [(work[w], w) for w in range(len(caps)) if len(bins[w]) < caps[w]]
    heapq.heapify(heap)
    for v in items[8 * units:]:
        wk, w = heapq.heappop(heap)
        bins[w].append(v)
        work[w] = wk + int(vlen[v])
        if len(bins[w]) < caps[w]:
            heapq.heappush(heap, (work[w], w))
    return bins


def _sweep_split_numpy(rowptr, cols, prev_rows, bands, piece=0, grid=None):
    """The sweep tables' rows restated: off[i][b] = row i's start plus its non-zeros with a column in the bands
    before b (band of column c: c * bands // prev_rows), off[i][bands] = its end.  Rows longer than the limit
    p (piece, or max(8, 3 x the mean + 10)) are split into m = ceil(len / p) pieces;
    piece i of m of row h takes [off[h][b] + n_b i // m, off[h][b] + n_b (i + 1) // m) of each band b.  range
    ((rows + pieces), 2 bands) holds each row's and then each piece's begin and end per band.  The initial order puts
    piece j at position (2 j + 1) npos // (2 pieces) and the unsplit rows in index order between; where that leaves
    some workgroup of 16 waves (grid workgroups, per = ceil(npos / (16 grid)) positions per wave) over 1.05 x the
    mean work (a piece's work: its row's length share len (i + 1) // m - len i // m), the rows and pieces are dealt
    to the waves, each of per positions (the last fewer), by _deal_numpy.  Returns range, the initial order, the
    split rows and split_ptr."""
    nr = len(rowptr) - 1
    lens = np.diff(rowptr)
    band = cols.astype(np.int64) * bands // prev_rows
    cnt = np.bincount(np.repeat(np.arange(nr), lens) * bands + band, minlength=nr * bands).reshape(nr, bands)
    off = np.empty((nr, bands + 1), np.int64)
    off[:, 0] = rowptr[:-1]
    off[:, 1:bands] = rowptr[:-1, None] + np.cumsum(cnt, axis=1)[:, :bands - 1]
    off[:, bands] = rowptr[1:]
    mean = int(rowptr[-1]) / nr
    limit = piece if piece > 0 else max(8, int(3.0 * mean + 10.0))
    psize = limit
    split = np.nonzero(lens > limit)[0]
    m = -(-lens[split] // psize)
    prow = np.repeat(split, m)
    pidx = np.concatenate([np.arange(k) for k in m]) if len(m) else np.zeros(0, np.int64)
    pcnt = np.repeat(m, m)
    npieces = len(prow)
    rng = np.empty((nr + npieces, 2 * bands), np.int64)
    rng[:nr, 0::2] = off[:, :bands]
    rng[:nr, 1::2] = off[:, 1:]
    o = off[prow, :bands]
    n = off[prow, 1:] - o
    rng[nr:, 0::2] = o + n * pidx[:, None] // pcnt[:, None]
    rng[nr:, 1::2] = o + n * (pidx + 1)[:, None] // pcnt[:, None]
    npos = nr - len(split) + npieces
    init = np.empty(npos, np.int64)
    at = (2 * np.arange(npieces) + 1) * npos // (2 * npieces) if npieces else np.zeros(0, np.int64)
    mask = np.zeros(npos, bool)
    mask[at] = True
    init[mask] = nr + np.arange(npieces)
    init[~mask] = np.setdiff1d(np.arange(nr), split)
    split_ptr = np.concatenate([[0], np.cumsum(m)])
    if grid is not None:
        vlen = np.concatenate([lens, lens[prow] * (pidx + 1) // pcnt - lens[prow] * pidx // pcnt]).astype(np.int64)
        per = -(-npos // (16 * grid))
        wg_pos = 16 * per
        n_wg = -(-npos // wg_pos)
        tot = np.add.reduceat(vlen[init], np.arange(0, npos, wg_pos))
        if int(tot.max()) * 20 * n_wg > int(tot.sum()) * 21:
            items = init[np.argsort(-vlen[init], kind="stable")]
            caps = [min(per, npos - w * per) for w in range(-(-npos // per))]
            for w, vs in enumerate(_deal_numpy(items, vlen, caps)):
                init[w * per: w * per + len(vs)] = vs
    return rng, init, split, split_ptr


def _sweep_tables_numpy(rowptr, cols, prev_rows, bands, per, steps=200, balance_steps=600, groups=None, paired=False,
                        piece=0, grid=None):
    """The swept step's tables restated (_sweep_split_numpy), then the order: each consecutive segment of `per`
    positions of the initial order longest first (the sum of its band ranges; ties by initial position), then, in
    segments of at most 64 positions, the plan's wave-parallel local search: at each of `steps` steps, each of 64
    lanes (xorshift32 per segment and lane) draws two positions; a pair whose swap can change a unit's rounds
    (different units, or with `paired` two lane groups of one pass) scores that change; the lowest score (ties:
    lowest lane) is applied when it adds no rounds.  `paired` counts units of two slots walked as one pass, as for a
    float32 sweep whose waves own over 24 rows.  Then each group of 16 segments (the waves of one workgroup) runs
    the plan's balance search over `balance_steps` steps (_balance_numpy).  Groups are independent: `groups`
    (indices) limits both searches to those, the others keep the sort.  Returns range, order, split, split_ptr."""
    rng, init, split, split_ptr = _sweep_split_numpy(rowptr, cols, prev_rows, bands, piece, grid)
    cnt = rng[:, 1::2] - rng[:, 0::2]                  # band counts of the rows and pieces
    lens = cnt.sum(axis=1)
    nr = len(init)                                     # positions
    order = np.empty(nr, np.int64)
    for b in range(0, nr, per):
        idx = np.arange(b, min(b + per, nr))
        order[b:b + len(idx)] = init[idx[np.lexsort((idx, -lens[init[idx]]))]]
    if per > 64 or steps == 0:
        return rng, order, split, split_ptr
    paired = bool(paired and bands == 4 and per > 24)
    U = 16 if paired else 8
    total_seg = -(-nr // per)
    n_groups = -(-total_seg // 16)
    groups = np.arange(n_groups) if groups is None else np.asarray(groups)
    segs = np.concatenate([np.arange(16 * g, min(16 * g + 16, total_seg)) for g in groups])
    nseg = len(segs)
    m = np.minimum(per, nr - segs * per)
    pad = np.full(total_seg * per, -1, np.int64)
    pad[:nr] = order
    rows = pad.reshape(total_seg, per)[segs]
    c = np.where(rows[:, None, :] >= 0, cnt[np.maximum(rows, 0)].transpose(0, 2, 1), 0)   # (nseg, bands, per)
    live = m > 8
    sg = segs.astype(np.uint64)[:, None]
    ln = np.arange(64, dtype=np.uint64)[None, :]
    low = np.uint64(0xFFFFFFFF)
    state = ((np.uint64(2463534242) ^ ((sg * np.uint64(2654435761)) & low) ^ (((ln + np.uint64(1)) * np.uint64(2246822507)) & low))
             | np.uint64(1)).astype(np.uint32)
    def nxt():
        nonlocal state
        state = state ^ (state << np.uint32(13))
        state = state ^ (state >> np.uint32(17))
        state = state ^ (state << np.uint32(5))
        return state
    seg_ix = np.arange(nseg)[:, None, None, None]
    band_ix = np.arange(bands)[None, None, :, None]
    def unit_cost(u, x, y):   # (nseg, L) -> rounds of unit u with the rows at positions x and y swapped
        r = np.clip(m[:, None] - U * u, 0, U)
        p = U * u[..., None] + np.arange(U)
        src = np.where(p == x[..., None], y[..., None], np.where(p == y[..., None], x[..., None], p))
        vals = c[seg_ix, band_ix, np.minimum(src, per - 1)[:, :, None, :]]                   # (nseg, L, bands, U)
        return np.where(r > 0, _unit_rounds_numpy(vals, r, paired), 0)
    us = np.tile(np.arange(8), (nseg, 1))
    cost = unit_cost(us, np.full_like(us, -1), np.full_like(us, -1))                          # (nseg, 8)
    ar = np.arange(nseg)
    for _ in range(steps):
        i = (nxt() % m[:, None].astype(np.uint32)).astype(np.int64)
        k = (nxt() % m[:, None].astype(np.uint32)).astype(np.int64)
        ui, uk = i // U, k // U
        ci, ck = unit_cost(ui, i, k), unit_cost(uk, i, k)
        cui, cuk = np.take_along_axis(cost, ui, 1), np.take_along_axis(cost, uk, 1)
        within = (ui == uk) & paired & ((i & 7) != (k & 7))
        d = np.where(ui != uk, ci + ck - cui - cuk, np.where(within, ci - cui, 1 << 20))
        w = np.argmin(((d + (1 << 20)) << 6) | np.arange(64)[None, :], axis=1)
        apply = live & (d[ar, w] <= 0)
        iw, kw = i[ar, w], k[ar, w]
        a = ar[apply]
        ia, ka = iw[apply], kw[apply]
        c[a, :, ia], c[a, :, ka] = c[a, :, ka].copy(), c[a, :, ia].copy()
        rows[a, ia], rows[a, ka] = rows[a, ka].copy(), rows[a, ia].copy()
        cost[a, ui[ar, w][apply]] = ci[ar, w][apply]
        cost[a, uk[ar, w][apply]] = ck[ar, w][apply]
    out = pad.reshape(total_seg, per).copy()
    out[segs] = rows
    order = out.reshape(-1)[:nr]
    if balance_steps:
        order = _balance_numpy(order, cnt, per, groups, balance_steps, paired)
    return rng, order, split, split_ptr


def test_sweep_band_table_order_and_rule_match_numpy():
    """The tables of a swept step (build_sweep, shared by the plan and the probe library's flyprobe_sweep_create):
    the range table of rows and split rows' pieces, the split rows, the initial order, the order of k_sweep_order,
    k_sweep_order_search and k_sweep_order_balance, and the size rule, against a numpy restatement, bit for bit, on
    random CSR matrices: 70,000 rows (18 rows per wave: slots of 8, 8 and 2) whose plain form sweeps and whose form
    with 32,768 source rows does not; the same with hub rows (longer than 3 x the mean + 10), which are split into
    pieces; 110,000 rows (27 per wave) searched for a float32 sweep that walks two slots per pass; and a forced
    piece size that splits a third of the rows.  The searches leave each workgroup its rows and pieces and each wave
    its number of positions, and lower the rounds and the workgroups' barrier-bound rounds on this fixed data."""
    import ctypes
    probe = ctypes.CDLL(os.path.join(REPO, "alpha-fly_amd", "csrc", "libflyprobe.so"))
    probe.flyprobe_last_error.restype = ctypes.c_char_p
    i64, i32, p_ = ctypes.c_int64, ctypes.c_int32, ctypes.c_void_p
    probe.flyprobe_sweep_create.argtypes = [p_, p_, i64, i64, i64, p_, ctypes.POINTER(p_), p_]
    probe.flyprobe_sweep_read.argtypes = [p_, p_, p_, p_, p_, p_, p_]
    probe.flyprobe_sweep_destroy.argtypes = [p_]
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    rng = np.random.default_rng(41)
    base_lens = rng.poisson(40, 70_000)
    hub = base_lens.copy()
    hub[12_345] = 4 * int(hub.mean()) + 200
    hub[70] = 3000
    hub[69_999] = 700
    clustered = np.sort(rng.poisson(40, 70_000) + rng.integers(0, 60, 70_000))[::-1].copy()   # long rows first
    cases = [("plain", 40_000, base_lens, 1, 0, (3, 4), 0), ("small source", 32_768, base_lens, 0, 0, (3, 4), 0),
             ("hub rows", 40_000, hub, 1, 0, (3, 4), 0), ("pairs", 40_000, rng.poisson(40, 110_000), 1, 1, (4,), 0),
             ("forced pieces", 40_000, base_lens, 1, 0, (4,), 44), ("clustered lengths", 40_000, clustered, 1, 0, (4,), 0)]
    for label, prev_rows, lens, want_swept, paired, band_counts, piece in cases:
        nr = len(lens)
        rowptr = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
        cols = np.concatenate([np.sort(rng.integers(0, prev_rows, n)) for n in lens]).astype(np.int32)
        pairs = np.stack([cols, rng.standard_normal(len(cols)).astype(np.float32).view(np.int32)], axis=1)
        d_rowptr = torch.as_tensor(rowptr, device=DEV)
        d_pairs = torch.as_tensor(np.ascontiguousarray(pairs), device=DEV)
        for bands in band_counts:
            cfg = (ctypes.c_int32 * 7)(bands, paired, 0, 0, piece, 1, 0)
            handle = p_()
            rc = probe.flyprobe_sweep_create(d_rowptr.data_ptr(), d_pairs.data_ptr(), nr, len(cols), prev_rows, cfg,
                                             ctypes.byref(handle), None)
            assert rc == 0, probe.flyprobe_last_error()
            print(f"{label}, {bands} bands: swept {bool(handle.value)}", flush=True)
            assert bool(handle.value) == bool(want_swept), (label, bands)
            if not want_swept:
                continue
            want_rng, init, want_split, want_ptr = _sweep_split_numpy(rowptr, cols, prev_rows, bands, piece, cus)
            npos, nv = len(init), len(want_rng)
            per = -(-npos // (16 * cus))
            nseg = -(-npos // per)
            ngrp = -(-nseg // 16)
            info = (ctypes.c_int64 * 7)()
            d_rng = torch.full((nv, 2 * bands), -7, dtype=torch.int32, device=DEV)
            d_order = torch.full((npos,), -7, dtype=torch.int32, device=DEV)
            d_split = torch.full((max(len(want_split), 1),), -7, dtype=torch.int32, device=DEV)
            d_ptr = torch.full((len(want_ptr),), -7, dtype=torch.int32, device=DEV)
            rc = probe.flyprobe_sweep_read(handle, info, d_rng.data_ptr(), d_order.data_ptr(), d_split.data_ptr(),
                                           d_ptr.data_ptr(), None)
            assert rc == 0, probe.flyprobe_last_error()
            probe.flyprobe_sweep_destroy(handle)
            torch.cuda.synchronize()
            assert list(info)[:6] == [npos, nv - nr, len(want_split), per, bands, cus], (label, list(info))
            assert np.array_equal(d_rng.cpu().numpy(), want_rng), (label, bands)
            if len(want_split):
                assert np.array_equal(d_split.cpu().numpy(), want_split) and np.array_equal(d_ptr.cpu().numpy(),
                                                                                            want_ptr), label
            print(f"  {len(want_split)} rows split into {nv - nr} pieces, {npos} positions, {per} per wave",
                  flush=True)
            check = np.r_[0:6, ngrp - 1]      # the searches restated for these groups of 16 waves (independent)
            _, order, _, _ = _sweep_tables_numpy(rowptr, cols, prev_rows, bands, per, groups=check,
                                                 paired=bool(paired), piece=piece, grid=cus)
            got = d_order.cpu().numpy()
            sel = np.concatenate([np.arange(16 * g * per, min(16 * (g + 1) * per, npos)) for g in check])
            assert np.array_equal(got[sel], order[sel]), (label, bands)
            _, sorted_order, _, _ = _sweep_tables_numpy(rowptr, cols, prev_rows, bands, per, steps=0,
                                                        balance_steps=0, piece=piece, grid=cus)
            for g0 in range(0, npos, 16 * per):
                assert np.array_equal(np.sort(got[g0:g0 + 16 * per]), np.sort(init[g0:g0 + 16 * per]))
            cnt = want_rng[:, 1::2] - want_rng[:, 0::2]
            U = 16 if paired and per > 24 else 8
            def cost(o):   # (rounds, barrier-bound rounds: per workgroup and band the largest wave's)
                m = np.minimum(per, npos - np.arange(nseg) * per)
                pad = np.full(nseg * per + U, -1, np.int64)
                pad[:npos] = o
                rows = np.stack([pad[np.arange(nseg) * per + j * U + np.arange(U)[:, None]].T
                                 for j in range(-(-per // U))], axis=1)               # (nseg, units, U)
                r = np.clip(m[:, None] - U * np.arange(rows.shape[1])[None, :], 0, U)
                rows = np.where(np.arange(U) < r[..., None], rows, -1)
                vals = np.where(rows[..., None] >= 0, cnt[np.maximum(rows, 0)], 0).transpose(0, 1, 3, 2)
                per_wave = np.stack([np.where(r > 0, _unit_rounds_numpy(vals[:, :, q:q + 1, :], r, U == 16), 0)
                                     .sum(axis=1) for q in range(bands)], axis=1)     # (nseg, bands)
                padw = np.zeros((ngrp * 16, bands), np.int64)
                padw[:nseg] = per_wave
                return int(per_wave.sum()), int(padw.reshape(ngrp, 16, bands).max(axis=1).sum())
            before, after = cost(sorted_order), cost(got)
            print(f"  rounds, barrier-bound rounds: longest first {before}, searched {after}", flush=True)
            assert after[0] < before[0] and after[1] < before[1], (label, bands, before, after)


def test_full_scale_b1120_deviation_agrees_with_float32(full_net):
    """The bench configuration: B = 1120 boards, float16 deviation vs float32 on the device."""
    from chessfly.synthetic import synthetic_boards
    net, _ = full_net
    x = torch.as_tensor(synthetic_boards(1120, seed=5)).to(DEV)
    out = {}
    for dtype in (torch.float32, torch.float16):
        net.infer_dtype = dtype
        with torch.no_grad():
            out[dtype] = net(x)
    net.infer_dtype = torch.float16
    (l32, w32), (l16, w16) = out[torch.float32], out[torch.float16]
    dl, dw = float((l16 - l32).abs().max()), float((w16 - w32).abs().max())
    agree = float((l16.argmax(1) == l32.argmax(1)).float().mean())
    print(f"B=1120: max |logit diff| {dl:.3e}, max |wdl diff| {dw:.3e}, argmax agreement {agree:.4%}", flush=True)
    assert dl < 1e-3 and dw < 1e-3 and agree >= 0.999


def _softmax_value(wdl: np.ndarray) -> np.ndarray:
    w = wdl.astype(np.float64)
    p = np.exp(w - w.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    return p[:, 0] - p[:, 2]


def _evaluator_outputs(lib, _hip, logits, wdl, rows=None, cols=None):
    batch, n_moves = logits.shape
    lg, wd = torch.as_tensor(logits, device=DEV), torch.as_tensor(wdl, device=DEV)
    values = torch.full((batch,), 7.0, device=DEV)
    bad = torch.full((1,), 5, dtype=torch.int32, device=DEV)             # the call clears it
    if rows is None:
        out = torch.zeros(batch, n_moves, dtype=torch.float16, device=DEV)
        args = (None, None, 0, out.data_ptr(), None)
    else:
        # an empty index list still needs non-null pointers: null rows selects the lazy form
        r, c = (torch.as_tensor(np.asarray(v, dtype=np.int64) if len(v) else np.zeros(1, np.int64), device=DEV)
                for v in (rows, cols))
        out = torch.zeros(len(rows), device=DEV)
        args = (r.data_ptr(), c.data_ptr(), len(rows), None, out.data_ptr())
    _hip.check(lib.fly_evaluator_outputs(lg.data_ptr(), wd.data_ptr(), batch, n_moves, *args, values.data_ptr(),
                                         bad.data_ptr(), _hip.stream(torch.device(DEV))), "fly_evaluator_outputs")
    return out.cpu().numpy(), values.cpu().numpy(), int(bad.item())


@pytest.mark.parametrize("batch,n_moves", [(37, 4168), (3, 5)])     # four-wide and one-wide conversion loops
def test_evaluator_outputs_kernel(batch, n_moves):
    """fly_evaluator_outputs against numpy: half rounding to nearest even (ties, overflow to inf, underflow,
    NaN), torch's wrapping of negative indices, flagged out-of-range indices, and the expected value against
    a float64 softmax (chessfly/model.py:107-110, 124-128)."""
    from chessfly import _hip
    lib = _hip.load()
    rng = np.random.default_rng(batch)
    logits = rng.normal(0, 4, (batch, n_moves)).astype(np.float32)
    logits.flat[:5] = [65504.0, 65520.0, -1e6, np.nan, 2.0 ** -25]        # max half, tie to inf, -inf, NaN, tie to 0
    logits.flat[-1] = 1.0 + 2.0 ** -11                                    # tie between 1 and 1 + 2^-10: rounds to 1
    wdl = rng.normal(0, 3, (batch, 3)).astype(np.float32)
    wdl[0] = [80.0, -80.0, 0.0]
    lazy, values, bad = _evaluator_outputs(lib, _hip, logits, wdl)
    want = logits.astype(np.float16)
    assert bad == 0
    assert np.array_equal(np.isnan(lazy), np.isnan(want))
    assert np.array_equal(lazy.view(np.uint16)[~np.isnan(want)], want.view(np.uint16)[~np.isnan(want)])
    assert np.isinf(lazy.flat[1]) and lazy.flat[2] == -np.inf and lazy.flat[4] == 0 and lazy.flat[-1] == 1
    np.testing.assert_allclose(values, _softmax_value(wdl), rtol=0, atol=1e-6)
    rows = np.concatenate([rng.integers(0, batch, 50), [-1, 0, -batch]])
    cols = np.concatenate([rng.integers(0, n_moves, 50), [-1, -n_moves, 2]])
    legal, values2, bad = _evaluator_outputs(lib, _hip, logits, wdl, rows, cols)
    want = logits[rows, cols]                                             # numpy wraps negatives as torch does
    assert bad == 0 and np.array_equal(legal.view(np.uint32), want.view(np.uint32))
    assert np.array_equal(values2, values)
    rows[3], cols[7] = batch, -n_moves - 1                                # out of range: NaN and the flag, no read
    legal, _, bad = _evaluator_outputs(lib, _hip, logits, wdl, rows, cols)
    assert bad == 1 and np.isnan(legal[3]) and np.isnan(legal[7])
    keep = np.ones(len(rows), dtype=bool)
    keep[[3, 7]] = False
    assert np.array_equal(legal[keep].view(np.uint32), want[keep].view(np.uint32))
    _, values3, bad = _evaluator_outputs(lib, _hip, logits, wdl, rows[:0], cols[:0])
    assert bad == 0 and np.array_equal(values3, values)


@pytest.mark.parametrize("nbytes", [4, 16, 100, 4100, 9_336_320])
def test_evaluator_download_copies_to_pinned_host_memory(nbytes):
    """fly_evaluator_download (the answers' copy to the host on a few CUs): every byte lands, for any length (16-byte
    pieces and a tail) and any workgroup count; a destination that is not pinned host memory, or a source that is
    not device memory, is refused, and the refusal leaves no error behind for the next call."""
    from chessfly import _hip
    lib = _hip.load()
    src = torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device=DEV)
    st = _hip.stream(torch.device(DEV))
    for wg in (0, 1, 3, 64):
        dst = torch.zeros(nbytes, dtype=torch.uint8, pin_memory=True)
        _hip.check(lib.fly_evaluator_download(src.data_ptr(), dst.data_ptr(), nbytes, wg, st), "fly_evaluator_download")
        torch.cuda.synchronize()
        assert torch.equal(dst, src.cpu()), wg
    plain = np.zeros(nbytes + 16, dtype=np.uint8)
    addr = plain.ctypes.data + (-plain.ctypes.data) % 16
    assert lib.fly_evaluator_download(src.data_ptr(), addr, nbytes, 0, st) != 0
    assert b"pinned host memory" in lib.fly_last_error()
    pinned_src = src.cpu().pin_memory()
    dst = torch.zeros(nbytes, dtype=torch.uint8, pin_memory=True)
    assert lib.fly_evaluator_download(pinned_src.data_ptr(), dst.data_ptr(), nbytes, 0, st) != 0
    assert b"source must be device memory" in lib.fly_last_error()
    assert lib.fly_evaluator_download(addr, dst.data_ptr(), nbytes, 0, st) != 0
    dst = torch.zeros(nbytes, dtype=torch.uint8, pin_memory=True)
    _hip.check(lib.fly_evaluator_download(src.data_ptr(), dst.data_ptr(), nbytes, 0, st), "fly_evaluator_download")
    torch.cuda.synchronize()
    assert torch.equal(dst, src.cpu())


def test_evaluator_protocol(full_net):
    """Evaluator.submit/result (chessfly/model.py:113-135): lazy fp16 policy vectors and eager legal gathers
    agree with FlyChessNet.forward on the same boards; several batches may be in flight at once."""
    from chessfly.model import Evaluator
    from chessfly.synthetic import synthetic_boards
    from chessfly.encoding import N_MOVES
    net, _ = full_net
    ev = Evaluator(net, torch.device(DEV))
    x = synthetic_boards(9, seed=2).astype(np.float16)
    with torch.no_grad():
        logits, wdl = (t.cpu().numpy() for t in net(torch.as_tensor(x, device=DEV).float()))
    lazy_logits, values = ev(x, None, None)
    assert lazy_logits.shape == (9, N_MOVES) and lazy_logits.dtype == np.float16 and values.shape == (9,)
    assert values.dtype == np.float32
    assert np.array_equal(lazy_logits.view(np.uint16), logits.astype(np.float16).view(np.uint16))
    np.testing.assert_allclose(values, _softmax_value(wdl), rtol=0, atol=1e-6)
    rows = np.repeat(np.arange(9), 5)
    cols = np.random.default_rng(0).integers(0, N_MOVES, size=45)
    first = ev.submit(x, rows, cols)                     # two batches in flight before either is read
    second = ev.submit(x[:4], None, None)
    legal, values2 = ev.result(first)
    lazy4, values4 = ev.result(second)
    assert legal.dtype == np.float32 and legal.shape == (45,)
    assert np.array_equal(legal, logits[rows, cols])
    assert np.array_equal(values2, values) and np.array_equal(values4, values[:4])
    assert np.array_equal(lazy4, lazy_logits[:4])
    assert np.all(np.abs(values) <= 1)
    legal0, values0 = ev(x, rows[:0], cols[:0])
    assert legal0.shape == (0,) and np.array_equal(values0, values)
    with pytest.raises(IndexError):
        ev(x, np.array([9]), np.array([0]))
    # six batches of different boards in flight (uploads, forwards and downloads on three streams): each
    # answer belongs to its own boards, bit for bit
    xs = [synthetic_boards(7 + i, seed=10 + i).astype(np.float16) for i in range(6)]
    handles = [ev.submit(xi, None, None) if i % 2 else ev.submit(xi, np.arange(len(xi)), np.arange(len(xi)))
               for i, xi in enumerate(xs)]
    for i, (xi, h) in enumerate(zip(xs, handles)):
        got, _ = ev.result(h)
        with torch.no_grad():
            want = net(torch.as_tensor(xi, device=DEV).float())[0].cpu().numpy()
        if i % 2:
            assert np.array_equal(got.view(np.uint16), want.astype(np.float16).view(np.uint16))
        else:
            assert np.array_equal(got, want[np.arange(len(xi)), np.arange(len(xi))])


def test_empty_batches_give_empty_outputs():
    """Zero boards through every public entry (as the reference's torch ops allow): empty outputs of the right
    shapes and dtypes, no launch errors, and the next non-empty call still correct."""
    from chessfly.encoding import N_FEATURES, N_MOVES
    from chessfly.model import Evaluator, FlyChessNet, ModelConfig
    from chessfly.synthetic import GraphSpec, synthetic_boards, synthetic_connectome
    conn = synthetic_connectome(GraphSpec(n=3000, edges=120_000, n_sensory=300, n_output=100, seed=4))
    torch.manual_seed(0)
    net = FlyChessNet(conn, ModelConfig(steps=4)).to(DEV).eval()
    rnn, n_in, n_out = net.brain, len(net.in_idx), len(net.out_idx)
    with torch.no_grad():
        for dtype in (torch.float32, torch.float16):
            out = rnn.forward_io(torch.zeros(n_in, 0, device=DEV, dtype=dtype), net.in_idx, net.out_idx, 4)
            assert out.shape == (n_out, 0) and out.dtype == torch.float32
            net.infer_dtype = dtype
            logits, wdl = net(torch.zeros(0, N_FEATURES, device=DEV))
            assert logits.shape == (0, N_MOVES) and wdl.shape == (0, 3)
        h = rnn(torch.zeros(conn.n_neurons, 0, device=DEV), 3)
        assert h.shape == (conn.n_neurons, 0)
        net.infer_dtype = torch.float16
        ev = Evaluator(net, torch.device(DEV))
        lazy, values = ev(np.zeros((0, N_FEATURES), np.float16), None, None)
        assert lazy.shape == (0, N_MOVES) and lazy.dtype == np.float16 and values.shape == (0,)
        legal, values = ev(np.zeros((0, N_FEATURES), np.float16), np.zeros(0, np.int64), np.zeros(0, np.int64))
        assert legal.shape == (0,) and values.shape == (0,)
        x = torch.as_tensor(synthetic_boards(5, seed=1), device=DEV)
        l5, _ = net(x)
        l1, _ = net(x[:1])
        torch.testing.assert_close(l5[:1], l1, rtol=0, atol=0)
    torch.cuda.synchronize()
