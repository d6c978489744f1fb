#!/usr/bin/env python3
"""Board-evals/s of the connectome network's forward evaluator on one MI355X.

Workload (default): the full-scale synthetic connectome (166,700 neurons, ~10.5M synapses), B = 1120 boards
(one leaf per concurrent self-play game), 6 recurrent steps through the light cone, float16 deviation from
the float32 resting trajectory, with the 838 -> 17,937 encoder and the 2,333 -> 4,168 policy / 3 WDL heads:
FlyChessNet.forward exactly as the search's Evaluator calls it, with the boards already on the device.

One "step" of this benchmark is one forward of the whole batch.  Prints one JSON line on stdout:
value = B * steps / wall time; `roofline` rates the fused state-step kernel by its compulsory HBM bytes
(CSR columns and values, per-row constants, previous/new state and input rows, read or written once) over
its launch time measured with HIP events on its stream; `roofline.replay` and `roofline.line_rate` set the
state step beside the replay of its own memory stream and beside the chip's rate of random 128-byte line reads
(libflyprobe.so); `cpu_baseline` times the reference's CPU path (restated in oracle/, the float32 light cone with
cached constants) on a bounded sample of the same boards.

    python bench.py [--steps K] [--warmup W] [--batch B] [--dtype f16|f32] [--graph synthetic|shuffled|realdeg]

`--graph realdeg` runs the same network on a graph with the MaleCNS wiring's in-degree sequence and sensory /
output sets (tests/golden/realdeg_fixture.npz, from the reference's shipped weight data) and seeded partners:
heavy-tailed in-degrees, hub rows of up to 9,193 partners, 2,190 neurons with none.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
for p in (REPO, os.path.join(REPO, "alpha-fly_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

METRIC = "board evals/sec, 6-step forward at B=1120; SpMM HBM GB/s vs peak"
HBM_PEAK_GBS = 8000.0


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def algorithmic_bytes(cone, batch: int, state_bytes: int) -> list[int]:
    """Compulsory bytes of each state-step launch t = 1..T: the CSR column (4 B) and value of every
    non-zero, the row pointer (4 B) and per-row constants (5 values) of every row, and the previous state,
    the new state and the input rows, each read or written once."""
    out = []
    for t in range(1, cone.steps + 1):
        nnz, rows, prev = cone.nnz[t], cone.row_counts[t], cone.row_counts[t - 1]
        fed = len(cone.u_pos[t])
        out.append(nnz * (4 + state_bytes) + (rows + 1) * 4 + rows * 5 * state_bytes
                   + batch * state_bytes * (prev + rows + fed))
    return out


def cpu_threads(requested: int = 0) -> tuple[int, int, str]:
    """Threads for the CPU baseline: len(os.sched_getaffinity(0)), capped at OMP_NUM_THREADS where the
    environment sets it (the CPU share a GPU job declares; a shared host's affinity mask can list cores other
    jobs use).  Returns (threads, affinity cores, a note on the choice)."""
    affinity = len(os.sched_getaffinity(0))
    if requested > 0:
        return requested, affinity, "--cpu-threads"
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and 0 < int(omp) < affinity:
        return int(omp), affinity, f"capped at OMP_NUM_THREADS={omp}"
    return affinity, affinity, "all affinity cores"


def cpu_baseline(net, conn, x_cpu, threads: int, prune: bool = True, seconds: float = 12.0):
    """The reference's CPU forward on the host cores: the float32 light cone with its constants cached per
    weight version (chessfly/brain.py:295-306), or with pruning off the literal recurrence
    (chessfly/brain.py:211-223); returns (evals/s, per-forward seconds, logits, wdl, repetitions)."""
    import warnings

    import numpy as np
    import torch

    warnings.filterwarnings("ignore", message="Sparse CSR tensor support is in beta")
    from chessfly.encoding import N_BASE, move_squares
    from chessfly.synthetic import synthetic_maps, synthetic_params
    from oracle import forward as F
    from oracle.lightcone import light_cone

    torch.set_num_threads(threads)
    p = synthetic_params(conn, seed=0)
    t = lambda a: torch.as_tensor(np.asarray(a, dtype=np.float32))
    w0 = F.normalised_weight(conn.n_neurons, conn.post, conn.syn_count) * p.global_scale
    ba = F.BrainArrays(conn.n_neurons, conn.pre, conn.post, conn.sign, w0, t(p.log_gain), t(p.bias), t(p.alpha_logit))
    in_idx, out_idx = conn.nodes("afferent").numpy(), conn.nodes("efferent").numpy()
    maps = synthetic_maps(len(in_idx), len(out_idx), 0)
    frm, to = move_squares()
    hp = F.HeadArrays(t(maps.encoder_w), t(maps.encoder_b), 5.0, N_BASE, t(maps.policy_w), t(maps.policy_b),
                      t(maps.from_w), t(maps.from_b), t(maps.to_w), t(maps.to_b), t(maps.value_w), t(maps.value_b),
                      torch.as_tensor(frm), torch.as_tensor(to), torch.zeros(len(out_idx)), torch.ones(len(out_idx)))
    cone = light_cone(conn.n_neurons, conn.pre.numpy(), conn.post.numpy(), in_idx, out_idx, net.cfg.steps)
    prep = F.prepare_f32(ba, cone)
    x = torch.as_tensor(x_cpu)
    steps = net.cfg.steps
    out_t = torch.as_tensor(out_idx)
    in_t = torch.as_tensor(in_idx)

    def forward():
        if prune:
            return F.model_forward(ba, hp, cone, x, "f32", prep=prep)
        u = torch.zeros(conn.n_neurons, x.shape[0]).index_copy_(0, in_t, F.encode_input(hp, x, torch.float32))
        return F.heads(hp, F.norm(hp, F.literal(ba, u, steps)[out_t].T))

    logits, wdl = forward()                                                   # warm-up
    times = []
    start = time.perf_counter()
    while len(times) < 3 or (time.perf_counter() - start < seconds and len(times) < 20):
        t0 = time.perf_counter()
        logits, wdl = forward()
        times.append(time.perf_counter() - t0)
    per = statistics.median(times)
    return x.shape[0] / per, per, logits, wdl, len(times)


def _train_targets(batch: int, dev, seed: int = 4):
    """Synthetic train_step targets (chessfly/train.py:113-124): ~30 legal moves per position with a visit
    distribution over them, and a WDL class."""
    import numpy as np
    import torch
    from chessfly.encoding import N_MOVES
    rng = np.random.default_rng(seed)
    legal = rng.random((batch, N_MOVES)) < 30 / N_MOVES
    legal[:, 0] = True
    pi = np.where(legal, rng.random((batch, N_MOVES)), 0.0)
    pi /= pi.sum(1, keepdims=True)
    t = lambda a, dt: torch.as_tensor(a, dtype=dt, device=dev)
    return t(pi, torch.float32), t(legal, torch.bool), t(rng.integers(0, 3, batch), torch.long)


def _train_loss(logits, wdl_logits, pi, legal, wdl):
    """policy_loss + value_loss of train_step with q_ratio 0 (chessfly/train.py:126-132)."""
    import torch.nn.functional as F
    logp = logits.masked_fill(~legal, -1e9).log_softmax(-1)
    return -(pi * logp).sum(-1).mean() + F.cross_entropy(wdl_logits, wdl)


def cpu_train_baseline(net, conn, x_cpu, threads: int, seconds: float = 15.0):
    """The reference's training forward + backward on the host cores (the float32 light cone under autograd
    with the CPU branch of _SparseRecurrent, chessfly/brain.py:66-99, 289-329; model.py:95-105), on the
    oracle's restatement with the net's current parameters; returns (positions/s, seconds, repetitions)."""
    import warnings

    import torch
    warnings.filterwarnings("ignore", message="Sparse CSR tensor support is in beta")
    from chessfly.encoding import N_BASE
    from oracle import forward as F
    from oracle import training as T
    from oracle.lightcone import light_cone

    torch.set_num_threads(threads)
    leaf = lambda p: p.detach().float().cpu().clone().requires_grad_(True)
    brain = net.brain
    w0 = F.normalised_weight(conn.n_neurons, conn.post, conn.syn_count) * net.cfg.weight_scale
    ba = F.BrainArrays(conn.n_neurons, conn.pre, conn.post, conn.sign, w0, leaf(brain.log_gain), leaf(brain.bias),
                       leaf(brain.alpha_logit))
    hp = F.HeadArrays(leaf(net.encoder.weight), leaf(net.encoder.bias), net.cfg.input_gain, N_BASE,
                      leaf(net.policy.weight), leaf(net.policy.bias), leaf(net.policy_from.weight),
                      leaf(net.policy_from.bias), leaf(net.policy_to.weight), leaf(net.policy_to.bias),
                      leaf(net.value.weight), leaf(net.value.bias), net.move_from.cpu(), net.move_to.cpu(),
                      net.norm.mean.cpu(), net.norm.var.cpu())
    cone = light_cone(conn.n_neurons, conn.pre.numpy(), conn.post.numpy(), net.in_idx.cpu().numpy(),
                      net.out_idx.cpu().numpy(), net.cfg.steps)
    x = torch.as_tensor(x_cpu)
    pi, legal, wdl = _train_targets(x.shape[0], "cpu")

    def step():
        logits, wdl_logits = T.model_grad(hp, ba, cone, x)
        _train_loss(logits, wdl_logits, pi, legal, wdl).backward()

    step()
    times = []
    start = time.perf_counter()
    while len(times) < 2 or (time.perf_counter() - start < seconds and len(times) < 10):
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
    per = statistics.median(times)
    return x.shape[0] / per, per, len(times)


def train_bench(args, dev) -> dict:
    """One train_step per step (chessfly/train.py:126-138): the float32 forward under autograd, the masked
    policy cross-entropy and value cross-entropy, backward, gradient clipping at 5 and an AdamW step, on the
    full synthetic graph at `--batch` positions."""
    import torch
    from chessfly import _hip
    from chessfly.synthetic import synthetic_boards, synthetic_net

    net, conn = bench_net(args, dev)
    net.train()
    opt = torch.optim.AdamW(net.parameters(), lr=1e-4, weight_decay=0.0)
    x_np = synthetic_boards(args.batch, seed=1)
    x = torch.as_tensor(x_np, dtype=torch.float32, device=dev)
    pi, legal, wdl = _train_targets(args.batch, dev)

    def step():
        logits, wdl_logits = net(x)
        loss = _train_loss(logits, wdl_logits, pi, legal, wdl)
        opt.zero_grad(set_to_none=True)
        loss.backward()
        torch.nn.utils.clip_grad_norm_(net.parameters(), 5.0)
        opt.step()
        return loss

    for _ in range(args.warmup):
        loss0 = step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        loss = step()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    # the device products' share from a shorter second pass with the library's launch events on
    prof_steps = min(args.steps, 5)
    _hip.profile_enable(True)
    for _ in range(prof_steps):
        step()
    torch.cuda.synchronize()
    prof = _hip.profile_read()
    _hip.profile_enable(False)
    value = args.batch * args.steps / wall
    sparse_ms = prof["other"][0] / prof_steps
    log(f"{args.steps} train steps: {wall * 1e3 / args.steps:.2f} ms each, {value:,.0f} positions/s; device sparse "
        f"products {sparse_ms:.2f} ms per step; loss {float(loss0):.4f} -> {float(loss):.4f}")
    cpu = None
    if args.cpu_boards > 0:
        nb = min(args.cpu_boards, args.batch, 64)
        threads, affinity, cap = cpu_threads(args.cpu_threads)
        log(f"CPU training baseline: {nb} positions on {threads} threads ({affinity} affinity cores; {cap}) ...")
        rate, per, reps = cpu_train_baseline(net, conn, x_np[:nb], threads)
        cpu = {"value": round(rate, 2), "unit": "positions/s", "cores": threads, "affinity_cores": affinity,
               "threads_note": cap, "kind": "port",
               "sample": f"{nb} positions, full graph, float32 light cone forward + backward under autograd "
                         f"(reference CPU path, chessfly/brain.py:66-99, 289-329), median of {reps} ({per:.2f} s each)"}
        log(f"CPU {rate:,.2f} positions/s")
    return {
        "metric": f"training positions/s (train_step: forward + backward + AdamW), B={args.batch}, "
                  f"{args.recurrent_steps} steps, fp32",
        "value": round(value, 1), "unit": "positions/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(wall * 1e3 / args.steps, 3), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": f"FlyChessNet train_step, synthetic connectome {conn.n_neurons} neurons / "
                               f"{conn.n_edges} synapses, B={args.batch}, {args.recurrent_steps} steps, light cone",
                   "batch": args.batch, "recurrent_steps": args.recurrent_steps, "graph": args.graph},
        "sparse_kernel_ms_per_step": round(sparse_ms, 3), "sparse_launches_per_step": prof["other"][1] // prof_steps,
        "cpu_baseline": cpu,
    }


REALDEG_FIXTURE = os.path.join(REPO, "tests", "golden", "realdeg_fixture.npz")


def realdeg_graph(seed: int = 0):
    """The graph with the MaleCNS wiring's in-degrees and sensory / output sets (the committed fixture) and
    partners drawn from `seed` (chessfly.synthetic.degree_connectome)."""
    import numpy as np
    from chessfly.synthetic import degree_connectome
    f = np.load(REALDEG_FIXTURE)
    ids = lambda gaps: np.cumsum(gaps.astype(np.int64))
    return degree_connectome(f["in_degree"], ids(f["in_idx_gaps"]), ids(f["out_idx_gaps"]), seed=seed)


def bench_net(args, dev):
    """The network of the benchmark's --graph on `dev`: the synthetic graph, its shuffled control, or the graph with
    the real in-degrees; the same seeded weights and maps either way."""
    from chessfly.synthetic import synthetic_net
    graph = realdeg_graph() if args.graph == "realdeg" else None
    return synthetic_net(steps=args.recurrent_steps, seed=0, shuffled=args.graph == "shuffled", device=dev,
                         graph=graph)


PROBE_LIB = os.path.join(REPO, "alpha-fly_amd", "csrc", "libflyprobe.so")


def _probe_lib():
    """libflyprobe.so (measurement probes, csrc/probe.hip), loaded with its argument types."""
    import ctypes
    if not os.path.exists(PROBE_LIB):
        raise RuntimeError(f"{PROBE_LIB} is missing: build it with `make -C alpha-fly_amd/csrc`")
    lib = ctypes.CDLL(PROBE_LIB)
    p, i32, i64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64
    lib.flyprobe_last_error.restype, lib.flyprobe_last_error.argtypes = ctypes.c_char_p, []
    for name, args in (("flyprobe_pack", [p, p, i64, p, p]),
                       ("flyprobe_sweep_create", [p, p, i64, i64, i64, p, ctypes.POINTER(p), p]),
                       ("flyprobe_sweep_destroy", [p]),
                       ("flyprobe_sweep_read", [p, p, p, p, p, p, p]),
                       ("flyprobe_replay_step", [p, p, i64, i64, p, i64, i64, i64, i32, p, p, p]),
                       ("flyprobe_pack_params", [p, p, i64, p, p]),
                       ("flyprobe_replay_step_io", [p, p, p, i64, i64, p, i64, i64, p, i64, i64, p, i64, i32, p, p]),
                       ("flyprobe_random_gather", [p, i64, i64, i64, p, i64, p, p]),
                       ("flyprobe_hashed_gather", [p, i64, i64, i64, i64, i64, i64, p, p]),
                       ("flyprobe_set_tuning", [ctypes.c_char_p, i64])):
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = i32, args
    return lib


def sweep_config(tuned: dict, state_f16: bool) -> list[int]:
    """The sweep tables' configuration a plan derives from its tuning (sweep_config in csrc/sweep.hpp): bands,
    paired, workgroups, force, piece, search, deal."""
    get = lambda k: int(tuned.get(k, 0))
    paired = get("sweep_paired") > 0
    return [3 if get("sweep_bands") == 3 else 4, int(paired), max(get("sweep_grid"), 0), int(get("swept") > 0),
            max(get("sweep_piece"), 0), int(get("sweep_order") >= 0), max(min(get("sweep_deal"), 1), -1)]


def _probe_check(lib, status: int, what: str) -> None:
    if status != 0:
        raise RuntimeError(f"{what} failed: {lib.flyprobe_last_error().decode(errors='replace')}")


def state_ld(batch: int, elem: int) -> int:
    """Row stride of the evaluator's state buffers (the batch rounded up to 64 columns, plus one 128-byte line
    when that leaves an even number of lines per row)."""
    line = 128 // elem
    ld = -(-batch // 64) * 64
    return ld + line if (ld // line) % 2 == 0 else ld


def _events_ms(fn, reps: int) -> float:
    """Average milliseconds of fn() over `reps` calls, between HIP events on torch's current stream (where fn
    launches)."""
    import torch
    fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


def issued_lines_per_nnz(rng, order, per: int, bands: int, paired: bool = False) -> float:
    """Lines a swept step's gathers issue per chunk of columns, per non-zero, from its tables (range (rows + pieces,
    2 bands), order (positions), rows_per_wave `per`): wave w takes positions [w per, (w + 1) per) in slots of 8;
    each slot issues, per band, 8 lane groups x its rounds: the longest of its rows' band counts (a slot of 3-4 rows
    spreads each row over 2 groups, of 2 rows over 4, of 1 row over 8, and the rounds run to the longest share),
    padded to a block of 4 rounds; a float32 sweep over pairs of slots runs each pass to the largest sum of a lane
    group's two rows (k_state_step_swept).  1.0: no padding gathers."""
    import numpy as np
    npos = len(order)
    cnt = (rng[:, 1::2] - rng[:, 0::2])[order].astype(np.int64)      # (npos, bands)
    nnz = int(cnt.sum())
    waves = -(-npos // per)
    unit = 16 if paired else 8
    units = -(-per // unit)
    full = np.zeros((waves, units * unit, bands), dtype=np.int64)
    have = np.zeros((waves, units * unit), dtype=bool)
    for w in range(waves):
        n = min(per, npos - w * per)
        full[w, :n] = cnt[w * per:w * per + n]
        have[w, :n] = True
    full = full.reshape(waves, units, unit, bands)
    have = have.reshape(waves, units, unit)
    if paired:
        rounds = (full[:, :, :8] + full[:, :, 8:]).max(axis=2)
    else:
        r = have.sum(axis=2)                                            # rows of each slot
        lf = np.where(r >= 5, 0, np.where(r >= 3, 1, np.where(r == 2, 2, 3)))
        share = (full + (1 << lf)[..., None, None] - 1) >> lf[..., None, None]
        rounds = share.max(axis=2)
    rounds = (rounds + 3) & ~3
    return float(8 * rounds.sum()) / max(nnz, 1)


def replay_ceiling(plan, cone, n_in: int, batch: int, state_f16: bool, dev, reps: int = 20,
                   tuned: dict | None = None) -> list[dict]:
    """Per step with a matrix, the time of the replay of that step's gather stream (flyprobe_replay_step: the
    state step's own kernel, launch shape and wave order over this plan's A_t and a state of this layout, with
    the arithmetic, row inputs and stores taken out), and of the replay that keeps the row reads and stores
    (flyprobe_replay_step_io: everything but the arithmetic of the sum)."""
    import torch
    from chessfly import _hip
    lib, probe = _hip.load(), _probe_lib()
    st = _hip.stream(dev)
    elem = 2 if state_f16 else 4
    ld = state_ld(batch, elem)
    dtype = torch.float16 if state_f16 else torch.float32
    sink = torch.empty(4096, dtype=torch.uint8, device=dev)
    out = []
    for t in range(1, cone.steps + 1):
        nr, nnz, prev_rows = cone.row_counts[t], cone.nnz[t], cone.row_counts[t - 1]
        if cone.ops[t] is None or nr == 0 or nnz == 0:
            continue
        rowptr = torch.empty(nr + 1, dtype=torch.int32, device=dev)
        col = torch.empty(nnz, dtype=torch.int32, device=dev)
        val = torch.empty(nnz, dtype=torch.float32, device=dev)
        _hip.check(lib.fly_plan_matrix(plan.handle, t, rowptr.data_ptr(), col.data_ptr(), val.data_ptr(), st),
                   "fly_plan_matrix")
        pairs = torch.empty(2 * nnz, dtype=torch.int32, device=dev)
        _probe_check(probe, probe.flyprobe_pack(col.data_ptr(), val.data_ptr(), nnz, pairs.data_ptr(), st),
                     "flyprobe_pack")
        del col, val
        xprev = (torch.randn(prev_rows, ld, device=dev) * 0.01).to(dtype)
        # where the evaluator sweeps this step, the probe replays the swept kernel over tables from the same builder
        # and configuration (the plan's tuning), which are then the plan's own
        import ctypes
        info = _hip.sweep_info(plan.handle, t)
        sweep = ctypes.c_void_p()
        if info["positions"]:
            cfg = (ctypes.c_int32 * 7)(*sweep_config(tuned or {}, state_f16))
            _probe_check(probe, probe.flyprobe_sweep_create(rowptr.data_ptr(), pairs.data_ptr(), nr, nnz, prev_rows,
                                                            cfg, ctypes.byref(sweep), st), "flyprobe_sweep_create")

        def once():
            _probe_check(probe, probe.flyprobe_replay_step(rowptr.data_ptr(), pairs.data_ptr(), nr, nnz,
                                                           xprev.data_ptr(), prev_rows, ld, batch, int(state_f16),
                                                           sweep, sink.data_ptr(), st),
                         "flyprobe_replay_step")
        row = {"t": t, "rows": nr, "nnz": nnz, "swept": bool(sweep.value), "replay_ms": round(_events_ms(once, reps), 4)}
        if info["pieces"]:
            row["split_rows"], row["pieces"] = info["split_rows"], info["pieces"]
        if sweep.value:
            sinfo = (ctypes.c_int64 * 7)()
            npos = info["positions"]
            d_rng = torch.empty((nr + info["pieces"], 2 * info["bands"]), dtype=torch.int32, device=dev)
            d_order = torch.empty(npos, dtype=torch.int32, device=dev)
            _probe_check(probe, probe.flyprobe_sweep_read(sweep, sinfo, d_rng.data_ptr(), d_order.data_ptr(), None,
                                                          None, st), "flyprobe_sweep_read")
            torch.cuda.synchronize()
            paired = bool(sinfo[6]) and not state_f16 and int((tuned or {}).get("sweep_paired", 0)) > 0
            row["issued_lines_per_nnz"] = round(issued_lines_per_nnz(d_rng.cpu().numpy(), d_order.cpu().numpy(),
                                                                     int(sinfo[3]), int(sinfo[4]), paired), 4)
            del d_rng, d_order
        # with the row I/O: each row's constants, carried state and input drive (float32, as the model forward's
        # encoder writes it) read, and the new state written
        prev32 = torch.empty(nr, dtype=torch.int32, device=dev)
        usrc32 = torch.empty(nr, dtype=torch.int32, device=dev)
        cone._step_export(t, prev=prev32, usrc=usrc32)
        params = torch.empty(nr * 8, dtype=torch.int32, device=dev)
        _probe_check(probe, probe.flyprobe_pack_params(prev32.data_ptr(), usrc32.data_ptr(), nr, params.data_ptr(), st),
                     "flyprobe_pack_params")
        ldu = state_ld(batch, 4)
        u = torch.randn(n_in, ldu, device=dev) * 0.01
        xout = torch.empty(nr, ld, dtype=dtype, device=dev)

        def once_io():
            _probe_check(probe, probe.flyprobe_replay_step_io(rowptr.data_ptr(), pairs.data_ptr(), params.data_ptr(),
                                                              nr, nnz, xprev.data_ptr(), prev_rows, ld, u.data_ptr(),
                                                              n_in, ldu, xout.data_ptr(), batch, int(state_f16),
                                                              sweep, st),
                         "flyprobe_replay_step_io")
        row["replay_io_ms"] = round(_events_ms(once_io, reps), 4)
        out.append(row)
        if sweep.value:
            probe.flyprobe_sweep_destroy(sweep)
        del rowptr, pairs, xprev, prev32, usrc32, params, u, xout
    return out


def random_gather_rates(dev, n: int = 1 << 26, reps: int = 5) -> tuple[dict, dict, dict]:
    """Context for the state step's gathers: GB/s of uniformly random 128-byte row reads in the state step's lane
    layout (8 rows per wave load, 16 bytes per lane) over working sets that fit one XCD's L2 (2 MB), that are one
    band of a swept step (41,600 rows: 5.3 MB), one 64-column chunk of 166,700 rows (21 MB, Infinity Cache) and
    neither (373 MB); rows per second over the 21 MB set for 128- and 64-byte reads.  The rows come from a hash with
    no index stream (flyprobe_hashed_gather): the chip's rate of random line reads.  The third dict repeats the sets
    with the row indices streamed from memory, one 4-byte load per read (flyprobe_random_gather): vector memory
    counters retire in order, so each index load from HBM holds up the reads issued after it, and that probe
    measures the latency of its own index stream."""
    import torch
    from chessfly import _hip
    probe = _probe_lib()
    sink = torch.zeros(256, device=dev)
    st = _hip.stream(dev)
    gbps, rows_per_s, indexed = {}, {}, {}
    sets = (("l2_2MB", 16384, 128), ("band_5MB", 41600, 128), ("infinity_cache_21MB", 166700, 128),
            ("hbm_373MB", 166700 * 35 // 2, 128), ("infinity_cache_21MB_64B", 166700, 64))
    for name, rows, read in sets:
        base = torch.randint(0, 256, (rows * 128,), dtype=torch.uint8, device=dev)

        def hashed():
            _probe_check(probe, probe.flyprobe_hashed_gather(base.data_ptr(), base.numel(), rows, 128, read, n, 12345,
                                                             sink.data_ptr(), st), "flyprobe_hashed_gather")
        sec = _events_ms(hashed, reps) * 1e-3
        if read == 128:
            gbps[name] = round(n * 128 / sec / 1e9, 1)
        if rows == 166700:
            rows_per_s[f"{read}B"] = round(n / sec / 1e9, 1)
        if read == 128:
            idx = torch.randint(0, rows, (n,), dtype=torch.int32, device=dev)

            def streamed():
                _probe_check(probe, probe.flyprobe_random_gather(base.data_ptr(), base.numel(), 128, read,
                                                                 idx.data_ptr(), n, sink.data_ptr(), st),
                             "flyprobe_random_gather")
            indexed[name] = round(n * 128 / (_events_ms(streamed, reps) * 1e-3) / 1e9, 1)
            del idx
        del base
    return gbps, rows_per_s, indexed


def evaluator_figure(net, dev, x_np, steps: int, legal_per_board: int = 32, download_workgroups: int = 0) -> dict:
    """The search's view (chessfly/model.py:113-135): fp16 boards from host numpy through Evaluator.submit
    and result, so the pinned H2D copy of the boards, the forward, the output kernel and the D2H copy of the
    answers are all inside the clock.  Lazy returns the whole fp16 policy; eager returns `legal_per_board`
    gathered logits per board.  "lazy"/"eager" run one batch at a time; "*_pipelined" keep two batches in
    flight, as the search's workers do (workers.py:118-167: submit the next batch, then take the previous
    result), so one batch's copies overlap the other's forward."""
    import numpy as np
    import torch
    from chessfly.encoding import N_MOVES
    import chessfly.model as model_mod
    from chessfly.model import Evaluator

    if download_workgroups > 0:
        model_mod.DOWNLOAD_SHARED = download_workgroups
    ev = Evaluator(net, dev)
    x16 = x_np.astype(np.float16)
    rng = np.random.default_rng(3)
    rows = np.repeat(np.arange(len(x16)), legal_per_board)
    cols = rng.integers(0, N_MOVES, size=len(rows))
    out = {}
    for name, r, c in (("lazy", None, None), ("eager", rows, cols)):
        ev(x16, r, c)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            ev.result(ev.submit(x16, r, c))
        dt = (time.perf_counter() - t0) / steps
        out[name] = {"evals_per_s": round(len(x16) / dt, 1), "ms_per_batch": round(dt * 1e3, 3)}
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        pending = ev.submit(x16, r, c)
        for _ in range(steps - 1):
            nxt = ev.submit(x16, r, c)
            ev.result(pending)
            pending = nxt
        ev.result(pending)
        dt = (time.perf_counter() - t0) / steps
        out[name + "_pipelined"] = {"evals_per_s": round(len(x16) / dt, 1), "ms_per_batch": round(dt * 1e3, 3)}
    out["note"] = (f"B={len(x16)} fp16 boards from host numpy, pinned staging; lazy: fp16 (B, {N_MOVES}) policy "
                   f"back; eager: {legal_per_board} legal logits per board back; plus values; pipelined: two "
                   f"batches in flight; the answers' download runs on {model_mod.DOWNLOAD_SHARED} workgroups while "
                   f"another batch computes, {model_mod.DOWNLOAD_ALONE} alone")
    return out


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30, help="timed forwards")
    ap.add_argument("--warmup", type=int, default=30)
    ap.add_argument("--batch", type=int, default=1120)
    ap.add_argument("--recurrent-steps", type=int, default=6)
    ap.add_argument("--dtype", choices=["f16", "f32"], default="f16")
    ap.add_argument("--graph", choices=["synthetic", "shuffled", "realdeg"], default="synthetic")
    ap.add_argument("--ones", default="40", help="ones per board: N or LO-HI")
    ap.add_argument("--no-prune", action="store_true",
                    help="compute every neuron at every step (the same function without the light cone)")
    ap.add_argument("--cpu-boards", type=int, default=256, help="boards in the CPU baseline sample (0: skip)")
    ap.add_argument("--train", action="store_true",
                    help="time the training step (forward + backward + AdamW, float32) instead of the evaluator; "
                         "--batch defaults to 256 here")
    ap.add_argument("--no-gather-ceiling", action="store_true",
                    help="skip the uniform random-row gather rates (context for the replay)")
    ap.add_argument("--no-replay", action="store_true",
                    help="skip the replay of each step's gather stream (the state step's ceiling)")
    ap.add_argument("--cpu-threads", type=int, default=0,
                    help="threads of the CPU baseline (0: the affinity cores, capped at OMP_NUM_THREADS when set)")
    ap.add_argument("--evaluator-steps", type=int, default=10,
                    help="batches through Evaluator.submit/result from host numpy, PCIe included (0: skip)")
    ap.add_argument("--tune", action="append", default=[], help="key=value for fly_set_tuning")
    ap.add_argument("--download-workgroups", type=int, default=0, metavar="N",
                    help="workgroups of the evaluator's answer download while another batch computes (0: the "
                         "evaluator's own choice, chessfly.model.DOWNLOAD_SHARED)")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="after the timed loop, run a plain float32 streaming copy of MIB MiB three times (a kernel "
                         "of known HBM traffic, to scale rocprof FETCH_SIZE / WRITE_SIZE readings)")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        msg = (f"bench.py measures one GPU: the evaluator shards by board across GPUs with no collective on the "
               f"critical path, and this evaluator runs on a single MI355X only (asked for --gpus {args.gpus}, "
               f"WORLD_SIZE {world})")
        print(msg, file=sys.stderr)
        print(msg)
        return 2

    import numpy as np
    import torch

    from chessfly import _hip
    from chessfly.synthetic import synthetic_boards, synthetic_net

    dev = torch.device("cuda:0")
    for kv in args.tune:
        k, v = kv.split("=")
        _hip.set_tuning(k, int(v))
    if args.train:
        if "--batch" not in sys.argv:
            args.batch = 256
        print(json.dumps(train_bench(args, dev)), flush=True)
        return 0
    t0 = time.perf_counter()
    net, conn = bench_net(args, dev)
    net.infer_dtype = torch.float16 if args.dtype == "f16" else torch.float32
    net.light_cone_pruning = not args.no_prune
    ones = tuple(int(v) for v in args.ones.split("-")) if "-" in args.ones else int(args.ones)
    x_np = synthetic_boards(args.batch, seed=1, ones=ones)
    x = torch.as_tensor(x_np, device=dev)
    torch.cuda.synchronize()
    log(f"graph {conn.n_neurons:,} neurons, {conn.n_edges:,} edges; net on {dev} in {time.perf_counter() - t0:.1f}s")

    brain = net.brain
    t0 = time.perf_counter()
    cone = brain.light_cone(net.in_idx, net.out_idx, args.recurrent_steps, prune=not args.no_prune)
    torch.cuda.synchronize()
    t_cone_first = time.perf_counter() - t0      # includes the process's first launches of the library
    from chessfly.brain import LightCone
    t0 = time.perf_counter()
    LightCone(brain, net.in_idx, net.out_idx, args.recurrent_steps, prune=not args.no_prune)
    torch.cuda.synchronize()
    t_cone = time.perf_counter() - t0
    mode = _hip.MODE_DEVIATION_F16 if args.dtype == "f16" else _hip.MODE_F32
    t0 = time.perf_counter()
    with torch.no_grad():
        brain._cone_plan(cone, mode)
    torch.cuda.synchronize()
    t_plan_first = time.perf_counter() - t0     # the cone's first plan: it also builds the steps' sweep tables
    # Later weight versions (as after each training phase) build a plan on the same cone and reuse its sweep
    # tables: a new version of the parameters with the same values, three times, the median kept.
    plan_times = []
    for _ in range(3):
        with torch.no_grad():
            brain.log_gain.add_(0.0)
            t0 = time.perf_counter()
            brain._cone_plan(cone, mode)
        torch.cuda.synchronize()
        plan_times.append(time.perf_counter() - t0)
    t_plan = statistics.median(plan_times)
    log(f"light cone {t_cone * 1e3:.1f} ms ({t_cone_first * 1e3:.1f} ms as the first library call), weight-set plan "
        f"{t_plan * 1e3:.1f} ms ({t_plan_first * 1e3:.1f} ms for the cone's first, with its sweep tables); rows "
        f"{cone.row_counts}, nnz {cone.nnz} ({cone.edge_visits:,} visits)")

    with torch.no_grad():
        for _ in range(args.warmup):
            net(x)
        torch.cuda.synchronize()
        stream = torch.cuda.current_stream(dev)
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        w0 = time.perf_counter()
        ev0.record(stream)
        for _ in range(args.steps):
            logits, wdl = net(x)
        ev1.record(stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - w0
        # the per-kernel-class split comes from a second pass with the library's launch events on, so the
        # timed pass above carries no measurement overhead
        _hip.profile_enable(True)
        for _ in range(args.steps):
            net(x)
        torch.cuda.synchronize()
        prof = _hip.profile_read()
        launches = _hip.profile_launches()
        _hip.profile_enable(False)
    if args.calibrate_copy > 0:
        src = torch.ones(args.calibrate_copy * 2**18, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.mul(src, 1.0, out=dst)
        torch.cuda.synchronize()
        log(f"calibration copy: 3 x {args.calibrate_copy} MiB read + {args.calibrate_copy} MiB written")
    gpu_ms = ev0.elapsed_time(ev1)
    ms_per_step = wall / args.steps * 1e3
    value = args.batch * args.steps / wall
    log(f"{args.steps} forwards: wall {wall * 1e3:.1f} ms, events {gpu_ms:.1f} ms -> {value:,.0f} evals/s; "
        f"kernel classes {prof}")

    state_bytes = 2 if args.dtype == "f16" else 4
    per_launch = algorithmic_bytes(cone, args.batch, state_bytes)
    step_ms, step_launches = prof["state_step"]
    launches_per_fwd = sum(1 for t in range(1, cone.steps + 1) if cone.row_counts[t] > 0)
    avg_launch_ms = step_ms / max(step_launches, 1)
    avg_bytes = sum(per_launch) / max(launches_per_fwd, 1)
    achieved = avg_bytes / (avg_launch_ms * 1e-3) / 1e9
    gather = sum(cone.nnz) * args.batch * state_bytes
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                "kernel": "k_state_step (fused CSR SpMM + input + clamp + leaky update)",
                "algorithmic_bytes_per_launch": int(avg_bytes), "launches_per_forward": launches_per_fwd,
                "avg_launch_ms": round(avg_launch_ms, 4),
                "gather_bytes_per_forward": int(gather),
                "gather_GBps": round(gather / (step_ms / max(step_launches, 1) * launches_per_fwd * 1e-3) / 1e9, 1)}
    # Traffic per launch comes from the rocprofv3 FETCH_SIZE / WRITE_SIZE passes committed beside the profile of
    # the same workload (counters cannot be read in-process); null for any other workload.  Those counters count
    # what leaves the L2 for the data fabric, which the 256 MB Infinity Cache or HBM then serves: gfx950 has no
    # counter that separates the two (TCC_EA0_RDREQ_DRAM counts every request "destined for DRAM", cache hits
    # included), so the figure is L2-to-fabric bytes, an upper bound on HBM bytes.
    traffic_file = os.path.join(REPO, "profiles", "state_step_b1120_traffic.json")
    if os.path.exists(traffic_file) and not args.tune:
        with open(traffic_file) as f:
            measured = json.load(f)
        here = {"batch": args.batch, "dtype": args.dtype, "prune": not args.no_prune, "graph": args.graph,
                "recurrent_steps": args.recurrent_steps, "ones": args.ones}
        if measured["workload"] == here:
            roofline["traffic"] = measured["traffic_bytes_per_launch"]
            roofline["traffic_kind"] = ("L2-to-fabric bytes per launch (calibrated FETCH_SIZE + WRITE_SIZE): served by "
                                        "the Infinity Cache or HBM, which no gfx950 counter separates")
            roofline["traffic_source"] = measured["source"]
    shares = {k: round(v[0] / args.steps, 4) for k, v in prof.items()}
    # per-step state-step times of the forward: the profiled pass's state-step launches, in step order
    step_launch_ms = [ms for cls, ms in launches if cls == "state_step"]
    live = [t for t in range(1, cone.steps + 1) if cone.row_counts[t] > 0]
    per_step = {t: statistics.mean(step_launch_ms[i::len(live)]) for i, t in enumerate(live)} \
        if len(step_launch_ms) == args.steps * len(live) else {}
    if not args.no_replay and per_step:
        # the ceiling: each step's own gather stream replayed alone (same kernel, shape and order, no arithmetic)
        plan = brain._cone_plan(cone, mode)
        tuned = dict(kv.split("=") for kv in args.tune)
        probe = _probe_lib()
        for key in ("sweep_paired", "sweep_slots", "sweep_pipe"):     # the swept kernel's launch-time choices
            if key in tuned:
                _probe_check(probe, probe.flyprobe_set_tuning(key.encode(), int(tuned[key])), "flyprobe_set_tuning")
        rows = replay_ceiling(plan, cone, len(net.in_idx), args.batch, args.dtype == "f16", dev, tuned=tuned)
        for r in rows:
            r["step_ms"] = round(per_step[r["t"]], 4)
            r["replay_over_step"] = round(r["replay_ms"] / r["step_ms"], 4)
            r["replay_io_over_step"] = round(r["replay_io_ms"] / r["step_ms"], 4)
        tot_replay = sum(r["replay_ms"] for r in rows)
        tot_io = sum(r["replay_io_ms"] for r in rows)
        tot_step = sum(r["step_ms"] for r in rows)
        roofline["replay"] = {
            "per_step": rows, "replay_ms": round(tot_replay, 4), "replay_io_ms": round(tot_io, 4),
            "step_ms": round(tot_step, 4),
            "frac_of_replay": round(tot_replay / tot_step, 4) if tot_step else None,
            "frac_of_replay_io": round(tot_io / tot_step, 4) if tot_step else None,
            "note": "replay = the state step's own kernel over the same A_t and state layout with the FMAs, row "
                    "inputs and stores taken out; replay_io = the same with the row reads and stores kept, i.e. "
                    "everything but the arithmetic of the sum (libflyprobe.so); frac_of_replay(_io) = replay time / "
                    "state-step time over the steps with a matrix (1.0: the step costs no more than that stream)"}
        log(f"replay of the gather stream: {tot_replay:.3f} ms, with the row I/O {tot_io:.3f} ms, against "
            f"{tot_step:.3f} ms of state steps (per step t, replay, replay_io, step: "
            f"{[(r['t'], r['replay_ms'], r['replay_io_ms'], r['step_ms']) for r in rows]})")
    if not args.no_gather_ceiling:
        rates, rows_per_s, indexed = random_gather_rates(dev)
        roofline["random_gather_GBps"] = rates
        roofline["random_gather_rows_per_s_21MB_G"] = rows_per_s
        roofline["random_gather_indexed_GBps"] = indexed
        log(f"uniform random-row gathers {rates} GB/s (index stream from memory: {indexed}); state step gathers at "
            f"{roofline['gather_GBps']} GB/s")
        # The line rate: the state step moves one 128-byte line of the previous state per non-zero and chunk of
        # columns (64 of the float16 state, 32 of float32); against the rate of uniformly random 128-byte reads
        # from an L2-resident set in the same lane layout with no index stream, the fastest such reads run on this
        # chip, and against the same reads over a set the size of one band of a swept step.
        per_line = 128 // state_bytes
        chunks = -(-args.batch // per_line)
        lines = sum(cone.nnz) * chunks
        step_fwd_ms = avg_launch_ms * launches_per_fwd
        probe = rates["l2_2MB"] * 1e9 / 128
        band = rates["band_5MB"] * 1e9 / 128
        line_rate = {"lines_per_forward": int(lines), "achieved_G_lines_per_s": round(lines / (step_fwd_ms * 1e-3) / 1e9, 2),
                     "l2_probe_G_lines_per_s": round(probe / 1e9, 2), "band_probe_G_lines_per_s": round(band / 1e9, 2),
                     "frac": round(lines / (step_fwd_ms * 1e-3) / probe, 4),
                     "frac_of_band_probe": round(lines / (step_fwd_ms * 1e-3) / band, 4), "per_step": []}
        for t, ms in per_step.items():
            n_t = cone.nnz[t] * chunks
            if n_t:
                line_rate["per_step"].append({"t": t, "lines": int(n_t), "ms": round(ms, 4),
                                              "G_lines_per_s": round(n_t / (ms * 1e-3) / 1e9, 2),
                                              "frac": round(n_t / (ms * 1e-3) / probe, 4),
                                              "frac_of_band_probe": round(n_t / (ms * 1e-3) / band, 4)})
        line_rate["note"] = ("gathered 128-byte lines (non-zeros x column chunks) per second of state step, against "
                             "uniformly random 128-byte reads in the same lane layout with no index stream "
                             "(flyprobe_hashed_gather) over a 2 MB (L2-resident) set (frac) and over a set the size of "
                             "one band of a swept step, 5.3 MB (frac_of_band_probe); frac stays on lines, roofline.frac "
                             "on algorithmic bytes")
        roofline["line_rate"] = line_rate
        log(f"line rate: {line_rate['achieved_G_lines_per_s']} G lines/s of state step against "
            f"{line_rate['l2_probe_G_lines_per_s']} for L2-resident random reads ({line_rate['frac']:.3f}); "
            f"per step {[(r['t'], r['G_lines_per_s'], r['frac']) for r in line_rate['per_step']]}")

    evaluator = None
    if args.evaluator_steps > 0:
        evaluator = evaluator_figure(net, dev, x_np, args.evaluator_steps,
                                     download_workgroups=args.download_workgroups)
        log(f"Evaluator from host numpy: {evaluator}")

    cpu = None
    parity = None
    if args.cpu_boards > 0:
        nb = min(args.cpu_boards, args.batch)
        threads, affinity, cap = cpu_threads(args.cpu_threads)
        log(f"CPU baseline: {nb} boards on {threads} threads ({affinity} affinity cores; {cap}) ...")
        rate, per, ref_logits, ref_wdl, reps = cpu_baseline(net, conn, x_np[:nb], threads, prune=not args.no_prune)
        path = ("float32 literal recurrence (reference CPU path, chessfly/brain.py:211-223)" if args.no_prune else
                "float32 light cone with cached constants (reference CPU path, chessfly/brain.py:295-329)")
        cpu = {"value": round(rate, 1), "unit": "board-evals/s", "cores": threads, "affinity_cores": affinity,
               "threads_note": cap, "kind": "port",
               "sample": f"{nb} of the {args.batch} boards, full graph, {path}, median of {reps} forwards "
                         f"({per:.2f} s each)"}
        dl = float((logits[:nb].float().cpu() - ref_logits).abs().max())
        dw = float((wdl[:nb].float().cpu() - ref_wdl).abs().max())
        agree = float((logits[:nb].argmax(1).cpu() == ref_logits.argmax(1)).float().mean())
        parity = {"boards": nb, "max_abs_logit": dl, "max_abs_wdl": dw, "argmax_agreement": agree,
                  "reference": "oracle float32 path"}
        log(f"CPU {rate:,.1f} evals/s; parity on {nb} boards: logits {dl:.2e}, wdl {dw:.2e}, argmax {agree:.4f}")

    line = {
        "metric": METRIC, "value": round(value, 1), "unit": "board-evals/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": (f"FlyChessNet.forward, {args.graph} connectome {conn.n_neurons} neurons / "
                                f"{conn.n_edges} synapses, B={args.batch}, {args.recurrent_steps} steps, "
                                + ("no pruning, " if args.no_prune else "light cone, ")
                                + ("fp16 deviation state, fp32 math" if args.dtype == "f16" else "fp32 state")),
                   "batch": args.batch, "recurrent_steps": args.recurrent_steps, "graph": args.graph,
                   "state": "fp16 deviation from fp32 resting trajectory" if args.dtype == "f16" else "fp32",
                   "light_cone": not args.no_prune, "edge_visits": cone.edge_visits, "rows": cone.row_counts[1:],
                   "ones_per_board": args.ones},
        "roofline": roofline, "cpu_baseline": cpu, "parity": parity,
        "kernel_ms_per_forward": shares, "gpu_event_ms_per_step": round(gpu_ms / args.steps, 4),
        "one_off_ms": {"light_cone": round(t_cone * 1e3, 1), "light_cone_first_call": round(t_cone_first * 1e3, 1),
                       "plan_first_with_sweep_tables": round(t_plan_first * 1e3, 1),
                       "plan": round(t_plan * 1e3, 1)},
        "evaluator": evaluator,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
