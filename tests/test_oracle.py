"""CPU tests: the oracle pinned against brute force, closed forms and the committed golden digests, plus the
product's host-side logic (connectome layout, shuffled control, move table).  No GPU needed."""

from __future__ import annotations

import json
import os
import warnings

import numpy as np
import pytest
import torch

from helpers import REPO, brain_arrays, random_params, tiny_connectome

from oracle import brute, lightcone as L, forward as F

warnings.filterwarnings("ignore", message="Sparse CSR tensor support is in beta")

GOLDEN = os.path.join(REPO, "tests", "golden", "fullscale_cone.json")


def _cone(conn, in_idx, out_idx, steps):
    return L.light_cone(conn.n_neurons, conn.pre.numpy(), conn.post.numpy(), in_idx, out_idx, steps)


TINY = [(120, 700, 3, np.arange(0, 9), np.arange(100, 120)),      # the reference's light-cone test graph
        (30, 200, 0, np.arange(0, 5), np.arange(25, 30)),
        (60, 600, 1, np.array([3, 7, 11, 40]), np.array([0, 7, 59]))]   # inputs and outputs overlapping


@pytest.mark.parametrize("n,e,seed,in_idx,out_idx", TINY)
@pytest.mark.parametrize("steps", [1, 2, 3, 4, 6])
def test_light_cone_rows_are_hop_distance_sets(n, e, seed, in_idx, out_idx, steps):
    conn = tiny_connectome(n, e, seed)
    cone = _cone(conn, in_idx, out_idx, steps)
    hop = brute.hop_cone(n, conn.pre.numpy(), conn.post.numpy(), in_idx, out_idx, steps)
    for t in range(steps + 1):
        assert cone.rows[t].tolist() == hop[t], t
    assert len(cone.rows[0]) == 0


@pytest.mark.parametrize("n,e,seed,in_idx,out_idx", TINY)
def test_light_cone_bookkeeping_by_definition(n, e, seed, in_idx, out_idx):
    conn = tiny_connectome(n, e, seed)
    steps = 5
    cone = _cone(conn, in_idx, out_idx, steps)
    pre, post = conn.pre.numpy(), conn.post.numpy()
    in_list = in_idx.tolist()
    for t in range(1, steps + 1):
        r_prev, r_next = cone.rows[t - 1].tolist(), cone.rows[t].tolist()
        op = cone.ops[t]
        if not r_prev:
            assert op is None
        else:
            edges, lrow, lcol = brute.brute_sub_matrix(pre, post, r_next, r_prev)
            assert op.edges.tolist() == edges and op.post.tolist() == lrow and op.pre.tolist() == lcol
            counts = np.bincount(np.asarray(lrow, dtype=np.int64), minlength=len(r_next))
            assert op.crow.tolist() == [0] + np.cumsum(counts).tolist()
            assert op.shape == (len(r_next), len(r_prev))
        for i, v in enumerate(r_next):
            carried = v in r_prev
            assert bool(cone.carried[t][i]) == carried
            assert cone.prev_row[t][i] == (r_prev.index(v) if carried else 0)
        assert cone.keep_next[t].tolist() == [i for i, v in enumerate(r_next) if v in r_prev]
        assert cone.keep_prev[t].tolist() == [r_prev.index(v) for v in r_next if v in r_prev]
        assert cone.u_pos[t].tolist() == [i for i, v in enumerate(r_next) if v in in_list]
        assert cone.u_src[t].tolist() == [in_list.index(v) for v in r_next if v in in_list]
    last = cone.rows[steps].tolist()
    assert cone.out_pos.tolist() == [j for j, v in enumerate(out_idx.tolist()) if v in last]
    assert cone.out_src.tolist() == [last.index(v) for v in out_idx.tolist() if v in last]
    assert cone.edge_visits == sum(len(op.edges) for op in cone.ops if op is not None)


def test_literal_matches_dense_closed_form_with_repeated_pairs():
    conn = tiny_connectome(40, 500, 2).shuffled(1)          # the control graph has repeated pairs and self-loops
    key = conn.post * conn.n_neurons + conn.pre
    assert len(torch.unique(key)) < len(key)
    lg, b, al = random_params(conn, 7, bias_sd=0.5)
    ba = brain_arrays(conn, 3.0, lg, b, al, dtype=torch.float64)
    u = torch.randn(conn.n_neurons, 6, dtype=torch.float64, generator=torch.Generator().manual_seed(0))
    W = brute.dense_matrix(conn.n_neurons, conn.pre.numpy(), conn.post.numpy(), F.edge_weights(ba, torch.float64).numpy())
    alpha = 1 / (1 + np.exp(-al.astype(np.float64)))
    for steps in (1, 2, 5):
        ref = brute.dense_recurrence(W, b.astype(np.float64), alpha, u.numpy(), steps)
        np.testing.assert_allclose(F.literal(ba, u, steps).numpy(), ref, rtol=1e-12, atol=1e-13)
        assert np.abs(ref).sum() > 0


def test_float16_literal_operands_are_the_rounded_weights():
    """literal_f16_operands (the reference's float16 literal recurrence, brain.py:213-216 with u float16): every weight
    and alpha is the float32 value rounded to nearest float16 (checked against numpy's float16 cast, and within half an
    ulp of float16), and the float64 recurrence over them is the dense closed form over those rounded values; with
    weights that are already float16 values it is the float32 operands' recurrence itself."""
    conn = tiny_connectome(40, 500, 2).shuffled(1)
    lg, b, al = random_params(conn, 11, bias_sd=0.5)
    ba = brain_arrays(conn, 3.0, lg, b, al)                       # float32 parameters, as the product's
    mat, alpha = F.literal_f16_operands(ba)
    w32 = F.edge_weights(ba, torch.float32).numpy()
    w16 = mat.values().numpy()
    np.testing.assert_array_equal(w16, w32.astype(np.float16).astype(np.float64))
    assert np.all(np.abs(w16 - w32) <= np.abs(w32) * 2.0 ** -11)
    a32 = (1 / (1 + np.exp(-al.astype(np.float64)))).astype(np.float32)
    np.testing.assert_allclose(alpha.numpy()[:, 0], a32.astype(np.float16).astype(np.float64), rtol=0, atol=1e-3)
    assert np.all(alpha.numpy()[:, 0] == alpha.numpy()[:, 0].astype(np.float16).astype(np.float64))
    W = brute.dense_matrix(conn.n_neurons, conn.pre.numpy(), conn.post.numpy(), w16)
    u = torch.randn(conn.n_neurons, 5, dtype=torch.float64, generator=torch.Generator().manual_seed(1))
    drive = u + torch.as_tensor(b, dtype=torch.float64)[:, None]
    h = torch.zeros_like(drive)
    for steps in range(1, 5):
        h = F.literal_step(ba, mat, alpha, h, drive)
        ref = brute.dense_recurrence(W, b.astype(np.float64), alpha.numpy()[:, 0], u.numpy(), steps)
        np.testing.assert_allclose(h.numpy(), ref, rtol=1e-12, atol=1e-13)


def test_unbounded_activity_matches_dense_closed_form():
    """h_max=None (brain.py:178-182, 221): the clamp keeps only its lower bound.  Biases large enough that
    activity passes 10, so a bound left in place would show; the light cone with h_max None is the same
    function as the literal recurrence."""
    conn = tiny_connectome(60, 900, 4).shuffled(2)
    lg, b, al = random_params(conn, 9, bias_mean=6.0, bias_sd=4.0)
    ba = brain_arrays(conn, 2.5, lg, b, al, h_max=None, dtype=torch.float64)
    u = torch.randn(conn.n_neurons, 4, dtype=torch.float64, generator=torch.Generator().manual_seed(3)) * 3
    W = brute.dense_matrix(conn.n_neurons, conn.pre.numpy(), conn.post.numpy(), F.edge_weights(ba, torch.float64).numpy())
    alpha = 1 / (1 + np.exp(-al.astype(np.float64)))
    for steps in (1, 3, 6):
        ref = brute.dense_recurrence(W, b.astype(np.float64), alpha, u.numpy(), steps, h_max=None)
        got = F.literal(ba, u, steps).numpy()
        np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-12)
        assert ref.max() > 10.0                       # the missing upper clamp matters here
        bounded = brute.dense_recurrence(W, b.astype(np.float64), alpha, u.numpy(), steps, h_max=10.0)
        assert np.abs(bounded - ref).max() > 1e-3
    in_idx, out_idx = np.arange(0, 8), np.arange(45, 60)
    for steps in (2, 5):
        cone = _cone(conn, in_idx, out_idx, steps)
        u_in = u[torch.as_tensor(in_idx)]
        full = torch.zeros_like(u).index_add(0, torch.as_tensor(in_idx), u_in)
        torch.testing.assert_close(F.cone_f32(ba, cone, u_in, steps),
                                   F.literal(ba, full, steps)[torch.as_tensor(out_idx)], rtol=1e-9, atol=1e-10)


def test_per_step_functions_compose_to_the_pinned_forwards():
    """literal_step, f32_step and deviation_step are the loop bodies of the pinned forwards: their states,
    collected step by step, end in the pinned outputs, and the first deviation step from d_0 = None matches
    its definition (s = input on input rows only, nothing carried)."""
    conn = tiny_connectome(120, 700, seed=3)
    lg, b, al = random_params(conn, 11)
    ba = brain_arrays(conn, 3.0, lg, b, al, dtype=torch.float64)
    in_idx, out_idx = np.arange(0, 9), np.arange(100, 120)
    steps = 4
    cone = _cone(conn, in_idx, out_idx, steps)
    u_in = torch.randn(9, 5, dtype=torch.float64, generator=torch.Generator().manual_seed(9))
    hs, ds = [], []
    out32 = F.cone_f32(ba, cone, u_in, steps)
    F.run_f32(F.prepare_f32(ba, cone, torch.float64), steps, u_in, states=hs)
    F.cone_half(ba, cone, u_in, steps, half=False, states=ds)
    assert [h.shape[0] for h in hs] == [len(cone.rows[t]) for t in range(1, steps + 1)]
    # deviation + resting trajectory = state, step by step (the deviation algebra, exact in float64)
    prep = F.prepare_f32(ba, cone, torch.float64)
    for t in range(1, steps + 1):
        c = prep["cs"][t][torch.as_tensor(cone.rows[t])]
        torch.testing.assert_close(ds[t - 1] + c, hs[t - 1], rtol=1e-10, atol=1e-12)
    last = torch.as_tensor(cone.out_src)
    torch.testing.assert_close(out32[torch.as_tensor(cone.out_pos)], hs[-1][last], rtol=0, atol=0)
    u = torch.zeros(conn.n_neurons, 5, dtype=torch.float64).index_add(0, torch.as_tensor(in_idx), u_in)
    mat, alpha = F.literal_operands(ba, torch.float64)
    drive = u + ba.bias.unsqueeze(1)
    h = torch.zeros_like(drive)
    for _ in range(steps):
        h = F.literal_step(ba, mat, alpha, h, drive)
    torch.testing.assert_close(h, F.literal(ba, u, steps), rtol=0, atol=0)


@pytest.mark.parametrize("steps", [1, 2, 4, 6])
def test_cone_forward_equals_literal_recurrence_fp64(steps):
    """The reference's light-cone invariant (tests/test_core.py:309-338): forward_io == forward[out_idx]."""
    conn = tiny_connectome(120, 700, seed=3)
    lg, b, al = random_params(conn, 11)
    ba = brain_arrays(conn, 3.0, lg, b, al, dtype=torch.float64)
    in_idx, out_idx = np.arange(0, 9), np.arange(100, 120)
    cone = _cone(conn, in_idx, out_idx, steps)
    u_in = torch.randn(9, 5, dtype=torch.float64, generator=torch.Generator().manual_seed(steps))
    u = torch.zeros(conn.n_neurons, 5, dtype=torch.float64).index_add(0, torch.as_tensor(in_idx), u_in)
    full = F.literal(ba, u, steps)[torch.as_tensor(out_idx)]
    torch.testing.assert_close(F.cone_f32(ba, cone, u_in, steps), full, rtol=1e-9, atol=1e-11)
    # the deviation algebra without float16 rounding is the same function
    torch.testing.assert_close(F.cone_half(ba, cone, u_in, steps, half=False), full, rtol=1e-9, atol=1e-11)
    # and so is the bookkeeping with pruning off (every neuron at every step)
    flat = L.light_cone(conn.n_neurons, conn.pre.numpy(), conn.post.numpy(), in_idx, out_idx, steps, prune=False)
    assert all(len(flat.rows[t]) == conn.n_neurons for t in range(1, steps + 1)) and len(flat.rows[0]) == 0
    torch.testing.assert_close(F.cone_f32(ba, flat, u_in, steps), full, rtol=1e-9, atol=1e-11)
    assert cone.edge_visits < 4 * conn.n_edges


@pytest.mark.parametrize("steps", [2, 6])
def test_float64_cone_over_a_float32_cache(steps):
    """float64 inputs to a float32 network (brain.py:295-306 with dtype float64): the cache is computed in the
    parameters' float32 and widened, so every cached value is a float32 and the float64 cone stays within the
    cache's float32 rounding of the exact function."""
    conn = tiny_connectome(120, 700, seed=3)
    lg, b, al = random_params(conn, 11)
    ba32 = brain_arrays(conn, 3.0, lg, b, al)
    ba64 = brain_arrays(conn, 3.0, lg, b, al, dtype=torch.float64)
    in_idx, out_idx = np.arange(0, 9), np.arange(100, 120)
    cone = _cone(conn, in_idx, out_idx, steps)
    prep = F.prepare_f32(ba32, cone, torch.float64, weights_dtype=torch.float32)
    for t in range(1, steps + 1):
        for v in (prep["cs"][t - 1], prep["ks"][t], prep["alpha"]) + \
                 ((prep["mats"][t].values(),) if prep["mats"][t] is not None else ()):
            assert v.dtype == torch.float64 and torch.equal(v.to(torch.float32).to(torch.float64), v)
    u_in = torch.randn(9, 5, dtype=torch.float64, generator=torch.Generator().manual_seed(steps))
    out = F.run_f32(prep, steps, u_in)
    assert out.dtype == torch.float64
    u = torch.zeros(conn.n_neurons, 5, dtype=torch.float64).index_add(0, torch.as_tensor(in_idx), u_in)
    exact = F.literal(ba64, u, steps)[torch.as_tensor(out_idx)]
    torch.testing.assert_close(out, exact, rtol=1e-5, atol=1e-5)
    assert (out - exact).abs().max() > 0          # the float32 cache does round


def test_deviation_algebra_on_clamped_rows_fp64():
    """Rows resting below 0 and above h_max: the clamp identity clamp(k+s,0,H) - clamp(k,0,H) =
    clamp(s,-k,H-k) + (k - clamp(k,0,H)) must hold exactly (brain.py:47-52)."""
    conn = tiny_connectome(200, 3000, seed=5)
    lg, b, al = random_params(conn, 3, gain_sd=0.8, bias_mean=0.6, bias_sd=0.7)
    b = b.copy()
    b[::17] += 12.0
    b[5::13] -= 3.0
    ba = brain_arrays(conn, 2.0, lg, b, al, dtype=torch.float64)
    in_idx, out_idx = np.arange(0, 40), np.arange(150, 200)
    for steps in (1, 3, 6):
        cone = _cone(conn, in_idx, out_idx, steps)
        u_in = torch.randn(40, 8, dtype=torch.float64, generator=torch.Generator().manual_seed(1)) * 0.5
        ref = F.cone_f32(ba, cone, u_in, steps)
        torch.testing.assert_close(F.cone_half(ba, cone, u_in, steps, half=False), ref, rtol=1e-10, atol=1e-12)


def test_half_emulation_within_reference_tolerance():
    """The reference's float16 acceptance test (tests/test_core.py:491-511) applied to the oracle's float16
    emulation: max |half - fp32| < 0.02 * signal + 1e-4 with a small signal on a large resting state."""
    conn = tiny_connectome(400, 9000, seed=5)
    g = torch.Generator().manual_seed(0)
    lg = (torch.randn(conn.n_edges, generator=g) * 0.8).numpy()
    b = (0.6 + torch.randn(conn.n_neurons, generator=g) * 0.7).numpy()
    b[::17] += 12.0
    al = torch.randn(conn.n_neurons, generator=g).numpy()
    ba = brain_arrays(conn, 2.0, lg, b, al)
    in_idx, out_idx = np.arange(0, 40), np.arange(300, 400)
    u = torch.randn(40, 64, generator=g) * 0.05
    for steps in (1, 3, 6):
        cone = _cone(conn, in_idx, out_idx, steps)
        ref = F.cone_f32(ba, cone, u, steps)
        half = F.cone_half(ba, cone, u, steps)
        signal = float((ref - ref.mean(1, keepdim=True)).abs().mean())
        assert float((half - ref).abs().max()) < 0.02 * signal + 1e-4


def test_heads_and_norm_closed_form():
    rng = np.random.default_rng(0)
    n_out, moves, batch = 17, 30, 4
    from oracle.forward import HeadArrays
    frm, to = rng.integers(0, 64, moves), rng.integers(0, 64, moves)
    t = lambda a: torch.as_tensor(np.asarray(a, dtype=np.float64))
    hp = HeadArrays(t(rng.normal(size=(5, 9))), t(rng.normal(size=5)), 5.0, 9,
                    t(rng.normal(size=(moves, n_out))), t(rng.normal(size=moves)),
                    t(rng.normal(size=(64, n_out))), t(rng.normal(size=64)),
                    t(rng.normal(size=(64, n_out))), t(rng.normal(size=64)),
                    t(rng.normal(size=(3, n_out))), t(rng.normal(size=3)),
                    torch.as_tensor(frm), torch.as_tensor(to),
                    t(rng.normal(size=n_out)), t(rng.uniform(0.001, 2, size=n_out)))
    r = t(rng.normal(size=(batch, n_out)) * 10)
    rn = F.norm(hp, r).numpy()
    P, W = hp, lambda a: a.numpy()
    for bi in range(batch):
        for j in range(n_out):
            z = (r[bi, j].item() - P.norm_mean[j].item()) / np.sqrt(P.norm_var[j].item() + 1e-8)
            assert rn[bi, j] == pytest.approx(min(max(z, -8.0), 8.0), rel=1e-12, abs=1e-12)
    logits, wdl = F.heads(hp, torch.as_tensor(rn))
    for bi in range(batch):
        for i in range(moves):
            want = (rn[bi] @ W(P.policy_w)[i] + W(P.policy_b)[i] + rn[bi] @ W(P.from_w)[frm[i]] + W(P.from_b)[frm[i]]
                    + rn[bi] @ W(P.to_w)[to[i]] + W(P.to_b)[to[i]])
            assert logits[bi, i].item() == pytest.approx(want, rel=1e-12, abs=1e-12)
        for k in range(3):
            assert wdl[bi, k].item() == pytest.approx(rn[bi] @ W(P.value_w)[k] + W(P.value_b)[k], rel=1e-12)
    p = np.exp(wdl.numpy()) / np.exp(wdl.numpy()).sum(1, keepdims=True)
    np.testing.assert_allclose(F.expected_value(wdl).numpy(), p[:, 0] - p[:, 2], rtol=1e-12)


def test_encode_input_closed_form():
    """encode_input (model.py:101-102: ((x[:, :n_base] W[:, :n_base]^T + b) * input_gain), cast, transposed) against a
    loop over the sensory rows: only the first n_base feature columns count (a change past them changes nothing), the
    gain multiplies the biased sum, the output is (n_in, B) contiguous in the requested dtype, and a float64 x is
    computed in float64."""
    rng = np.random.default_rng(5)
    from oracle.forward import HeadArrays
    n_in, k_all, n_base, batch = 7, 12, 9, 5
    t = lambda a: torch.as_tensor(np.asarray(a, dtype=np.float64))
    z = lambda *shape: t(np.zeros(shape))
    hp = HeadArrays(t(rng.normal(size=(n_in, k_all))), t(rng.normal(size=n_in)), 5.0, n_base, z(3, 2), z(3), z(64, 2),
                    z(64), z(64, 2), z(64), z(3, 2), z(3), torch.zeros(3, dtype=torch.long),
                    torch.zeros(3, dtype=torch.long), z(2), t(np.ones(2)))
    x = t(rng.integers(0, 2, size=(batch, k_all)))
    u = F.encode_input(hp, x, torch.float64)
    assert u.shape == (n_in, batch) and u.is_contiguous() and u.dtype == torch.float64
    W, b = hp.enc_w.numpy(), hp.enc_b.numpy()
    for i in range(n_in):
        for bi in range(batch):
            want = (sum(x[bi, f].item() * W[i, f] for f in range(n_base)) + b[i]) * 5.0
            assert u[i, bi].item() == pytest.approx(want, rel=1e-13, abs=1e-13)
    x2 = x.clone()
    x2[:, n_base:] = 1.0 - x2[:, n_base:]
    assert torch.equal(F.encode_input(hp, x2, torch.float64), u), "columns past n_base must not count"
    u16 = F.encode_input(hp, x.float(), torch.float16)   # float32 arithmetic, then one float16 rounding
    assert u16.dtype == torch.float16 and u16.shape == (n_in, batch)
    assert float((u16.double() - u).abs().max()) <= float(u.abs().max()) * 2.0 ** -10


def test_move_squares_matches_the_move_index_of_every_move():
    """move_squares against the policy-index definition (chessfly/encoding.py:70-77) for every normal move
    and every legal underpromotion (the check of tests/test_core.py:394-405, without python-chess)."""
    from chessfly.encoding import N_MOVES, move_squares
    frm, to = move_squares()
    assert frm.shape == to.shape == (N_MOVES,)
    for f in range(64):
        for t in range(64):
            i = f * 64 + t
            assert (frm[i], to[i]) == (f, t)
    seen = set()
    for ff in range(8):
        for tf in (ff - 1, ff, ff + 1):
            if not 0 <= tf <= 7:
                continue
            for piece in range(3):                      # knight, bishop, rook
                i = 4096 + (ff * 3 + (tf - ff + 1)) * 3 + piece
                seen.add(i)
                assert (frm[i], to[i]) == (48 + ff, 56 + tf)
    assert len(seen) == 66 and max(seen) < N_MOVES


def test_shuffled_keeps_degrees_and_dale():
    """tests/test_core.py:64-71 on the product's Connectome.shuffled."""
    c = tiny_connectome()
    s = c.shuffled()
    assert torch.equal(torch.bincount(s.post, minlength=30), torch.bincount(c.post, minlength=30))
    assert torch.equal(torch.bincount(s.pre, minlength=30), torch.bincount(c.pre, minlength=30))
    nt_sign = torch.ones(30).index_put_((c.pre,), c.sign)
    assert torch.equal(s.sign, nt_sign[s.pre])
    assert torch.all(s.post[1:] >= s.post[:-1])
    key = s.post * 30 + s.pre
    assert torch.all(key[1:] >= key[:-1])                  # (post, pre) order


def test_connectome_weight_normalises_inputs():
    c = tiny_connectome(50, 400, 4)
    w = c.weight
    sums = torch.zeros(50).index_add_(0, c.post, w)
    has_input = torch.bincount(c.post, minlength=50) > 0
    torch.testing.assert_close(sums[has_input], torch.ones(int(has_input.sum())))


def test_synthetic_boards():
    from chessfly.synthetic import synthetic_boards
    from chessfly.encoding import N_BASE, N_FEATURES
    x = synthetic_boards(50, seed=3)
    assert x.shape == (50, N_FEATURES) and set(np.unique(x)) <= {0.0, 1.0}
    assert (x[:, :N_BASE].sum(1) == 40).all() and x[:, N_BASE:].sum() == 0
    y = synthetic_boards(200, seed=4, ones=(20, 40))
    counts = y.sum(1)
    assert counts.min() >= 20 and counts.max() <= 40 and len(np.unique(counts)) > 5
    np.testing.assert_array_equal(synthetic_boards(50, seed=3), x)


@pytest.mark.slow
def test_full_scale_synthetic_graph_and_oracle_cone_match_golden():
    """The seeded generator and the oracle's full-scale cone reproduce the committed digests."""
    from golden.make_golden import cone_record, graph_record
    from chessfly.synthetic import FULL, synthetic_connectome, synthetic_params
    with open(GOLDEN) as f:
        gold = json.load(f)
    conn = synthetic_connectome(FULL)
    assert graph_record(conn) == {k: v for k, v in gold["graphs"]["synthetic"].items() if k != "cones"}
    assert synthetic_params(conn, seed=0).global_scale == gold["global_scale"]
    cone = _cone(conn, conn.nodes("afferent").numpy(), conn.nodes("efferent").numpy(), 6)
    assert cone_record(cone) == gold["graphs"]["synthetic"]["cones"]["6"]
