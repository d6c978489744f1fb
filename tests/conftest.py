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
