import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a real MI355X (HIP device)")
    config.addinivalue_line("markers", "slow: long-running CPU test")


def gpu_available() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def default_params():
    """The default-dims weights (init spec, seed 0; 2 B values, 8 GB on the
    host), generated once per session for every test that needs them."""
    from hackathon_amd import spec, weights

    return weights.generate(spec.DEFAULT, 0)


@pytest.fixture(scope="session")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    return torch.device("cuda:0")


def pytest_runtest_logstart(nodeid, location):
    # Name the case before any GPU step, so a box that dies mid-run still says
    # which test it was on.
    if os.environ.get("HK_ANNOUNCE", "1") == "1":
        print(f"\n[start] {nodeid}", flush=True)
