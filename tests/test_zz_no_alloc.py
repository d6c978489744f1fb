"""fly_model_forward_static, the model forward that allocates nothing (its scratch is a static device array), against
fly_model_forward with a torch workspace, through the C ABI: two calls in a row, the second smaller, in both state
dtypes, on the full-scale network (so the static entry point runs its batch as several blocks)."""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _forward(lib, _hip, plan, dense, x, static: bool):
    batch = x.shape[0]
    logits = torch.full((batch, 4168), float("nan"), device=DEV)
    wdl = torch.full((batch, 3), float("nan"), device=DEV)
    st = _hip.stream(torch.device(DEV))
    if static:
        _hip.check(lib.fly_model_forward_static(plan.handle, dense.handle, x.data_ptr(), 0, x.stride(0), batch, 5.0,
                                                logits.data_ptr(), wdl.data_ptr(), st), "fly_model_forward_static")
    else:
        ws = _hip.workspace(lib.fly_model_workspace(plan.handle, dense.handle, batch), x.device)
        _hip.check(lib.fly_model_forward(plan.handle, dense.handle, x.data_ptr(), 0, x.stride(0), batch, 5.0,
                                         logits.data_ptr(), wdl.data_ptr(), ws.data_ptr(), ws.numel(), st),
                   "fly_model_forward")
    torch.cuda.synchronize()
    return logits, wdl


def test_static_scratch_forward_matches_the_workspace_forward(full_net):
    from chessfly import _hip
    from chessfly.encoding import N_BASE
    from chessfly.synthetic import synthetic_boards
    lib = _hip.load()
    net, _ = full_net
    brain = net.brain
    cone = brain.light_cone(net.in_idx, net.out_idx, net.cfg.steps)
    dense = net._dense(N_BASE)
    x_all = torch.as_tensor(synthetic_boards(600, seed=51)).to(DEV)
    for mode, tol in ((_hip.MODE_DEVIATION_F16, 1e-3), (_hip.MODE_F32, 5e-5)):
        with torch.no_grad():
            plan = brain._cone_plan(cone, mode)
        # 600 boards: blocks of 256 (float16 state) or 128 (float32); then 100 boards, one block, over the array's
        # leftovers from the larger call
        for batch in (600, 100):
            x = x_all[:batch]
            ref = _forward(lib, _hip, plan, dense, x, static=False)
            got = _forward(lib, _hip, plan, dense, x, static=True)
            for a, b in zip(got, ref):
                assert bool(torch.isfinite(a).all())
                d = float((a - b).abs().max())
                print(f"mode {mode} B={batch}: max |static - workspace| {d:.3e}", flush=True)
                assert d < tol, (mode, batch, d)
            assert torch.equal(got[0].argmax(1), ref[0].argmax(1))


def test_static_scratch_refuses_what_does_not_fit_and_bad_arguments():
    """A network whose one block of 64 boards needs more than the static array is refused with a clear error before
    anything is launched: 400,000 neurons without the light cone, float32 state (two 400,000 x 96 float32 state
    buffers, 307 MB); its float16 deviation state (102 MB) runs.  Null pointers are refused too."""
    from chessfly import _hip
    from chessfly.encoding import N_BASE
    from chessfly.synthetic import GraphSpec, synthetic_boards, synthetic_net
    lib = _hip.load()
    assert lib.fly_model_forward_static(None, None, None, 0, 838, 4, 5.0, None, None, None) == 1
    assert b"null" in lib.fly_last_error()
    spec = GraphSpec(n=400_000, edges=1_000_000, n_sensory=1000, n_output=100, seed=3)
    net, _ = synthetic_net(spec, steps=3, seed=0, device=DEV)
    cone = net.brain.light_cone(net.in_idx, net.out_idx, 3, prune=False)
    dense = net._dense(N_BASE)
    x = torch.as_tensor(synthetic_boards(64, seed=52)).to(DEV)
    logits = torch.empty(64, 4168, device=DEV)
    wdl = torch.empty(64, 3, device=DEV)
    st = _hip.stream(torch.device(DEV))
    with torch.no_grad():
        p32 = net.brain._cone_plan(cone, _hip.MODE_F32)
        p16 = net.brain._cone_plan(cone, _hip.MODE_DEVIATION_F16)
    rc = lib.fly_model_forward_static(p32.handle, dense.handle, x.data_ptr(), 0, x.stride(0), 64, 5.0,
                                      logits.data_ptr(), wdl.data_ptr(), st)
    assert rc == 1 and b"static array" in lib.fly_last_error(), lib.fly_last_error()
    ref = _forward(lib, _hip, p16, dense, x, static=False)
    got = _forward(lib, _hip, p16, dense, x, static=True)
    assert float((got[0] - ref[0]).abs().max()) < 1e-3 and float((got[1] - ref[1]).abs().max()) < 1e-3


def test_static_forward_allocates_nothing_and_runs_under_graph_capture(full_net):
    """The property the entry point exists for.  A warm call leaves the device's free memory unchanged, and one call
    captured into a HIP graph (capture fails if the call allocates, frees or synchronises) replays correctly: three
    replays with new boards copied in and the workspace forward run eagerly between them, each replay's outputs
    within 1e-3 of that forward's (float16 state, 300 boards: two blocks of the static array)."""
    from chessfly import _hip
    from chessfly.encoding import N_BASE
    from chessfly.synthetic import synthetic_boards
    lib = _hip.load()
    net, _ = full_net
    cone = net.brain.light_cone(net.in_idx, net.out_idx, net.cfg.steps)
    dense = net._dense(N_BASE)
    with torch.no_grad():
        plan = net.brain._cone_plan(cone, _hip.MODE_DEVIATION_F16)
    batch = 300
    x = torch.as_tensor(synthetic_boards(batch, seed=60)).to(DEV)
    logits = torch.zeros(batch, 4168, device=DEV)
    wdl = torch.zeros(batch, 3, device=DEV)

    def call():
        _hip.check(lib.fly_model_forward_static(plan.handle, dense.handle, x.data_ptr(), 0, x.stride(0), batch, 5.0,
                                                logits.data_ptr(), wdl.data_ptr(), _hip.stream(torch.device(DEV))),
                   "fly_model_forward_static")

    call()                                   # first call on the device: looks up the static array's address
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    call()
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info()[0] == free0
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call()
    torch.cuda.synchronize()
    for i in range(3):
        x.copy_(torch.as_tensor(synthetic_boards(batch, seed=61 + i)).to(DEV))
        logits.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        got = (logits.clone(), wdl.clone())
        ref = _forward(lib, _hip, plan, dense, x, static=False)
        for a, b in zip(got, ref):
            d = float((a - b).abs().max())
            print(f"replay {i}: max |graph replay - workspace forward| {d:.3e}", flush=True)
            assert bool(torch.isfinite(a).all()) and d < 1e-3, (i, d)
