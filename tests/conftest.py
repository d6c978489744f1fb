import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (REPO, os.path.join(REPO, "alpha-fly_amd"), os.path.join(REPO, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X) and the built libflyeval.so")
    config.addinivalue_line("markers", "slow: full-scale graph (166,700 neurons); minutes on the CPU")


def pytest_collection_modifyitems(config, items):
    import torch
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no HIP device in this process")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def full_net():
    """The full-scale synthetic network on cuda:0 and its Connectome (built once per session)."""
    import torch
    from chessfly.synthetic import synthetic_net
    net, conn = synthetic_net(steps=6, seed=0, device="cuda:0")
    torch.cuda.synchronize()
    return net, conn


# Tuning under which the small-graph oracle tests run the banded sweep: plans capture the tuning when they are
# created, so the fixture sets it before the test builds its network and resets it afterwards.  "swept" sweeps every
# step with a matrix at one workgroup per CU (a row or two per wave: rows spread over lane groups); fewer
# workgroups give each wave passes of 6 slots ("4wg": about 47 rows per wave on a 3,000-neuron graph), several passes
# ("2wg"), split rows whose pieces meet in the finish kernel ("pieces"), paired passes, passes of 3 slots with the
# next gathers in flight, 3 bands and the unsearched order.
SWEEP_MODES = {
    "auto": {},
    "swept": {"swept": 1},
    "swept-4wg": {"swept": 1, "sweep_grid": 4},
    "swept-2wg-pieces": {"swept": 1, "sweep_grid": 2, "sweep_piece": 24},
    "swept-4wg-paired": {"swept": 1, "sweep_grid": 4, "sweep_paired": 1},
    "swept-4wg-3slots-pipe": {"swept": 1, "sweep_grid": 4, "sweep_slots": 3},
    "swept-8wg-3bands-unsearched": {"swept": 1, "sweep_grid": 8, "sweep_bands": 3, "sweep_order": -1},
}


@pytest.fixture(params=list(SWEEP_MODES))
def sweep_mode(request):
    from chessfly import _hip
    keys = SWEEP_MODES[request.param]
    for k, v in keys.items():
        _hip.set_tuning(k, v)
    try:
        yield request.param
    finally:
        for k in keys:
            _hip.set_tuning(k, 0)


def swept_steps(plan_handle, steps: int) -> list:
    """The steps of a plan that run as a banded sweep (fly_plan_sweep_info), with their positions and pieces."""
    from chessfly import _hip
    out = []
    for t in range(1, steps + 1):
        info = _hip.sweep_info(plan_handle, t)
        if info["positions"]:
            out.append((t, info["positions"], info["pieces"], info["workgroups"]))
    return out


SWEEP_CORE = ["auto", "swept-4wg", "swept-2wg-pieces", "swept-4wg-paired"]


@pytest.fixture(params=SWEEP_CORE)
def sweep_core(request):
    """sweep_mode over a subset: the default, passes of 6 slots, split rows over several passes, paired passes."""
    from chessfly import _hip
    keys = SWEEP_MODES[request.param]
    for k, v in keys.items():
        _hip.set_tuning(k, v)
    try:
        yield request.param
    finally:
        for k in keys:
            _hip.set_tuning(k, 0)
