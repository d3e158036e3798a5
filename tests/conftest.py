import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")
    config.addinivalue_line("markers", "slow: CPU test that takes more than a few seconds")


@pytest.fixture(scope="session")
def hip_ctx():
    """One HIP context for all GPU tests (created only when a GPU test runs)."""
    from alpaca_amd.model import HIPContext
    ctx = HIPContext(0)
    yield ctx
    ctx.close()


@pytest.fixture(scope="session")
def hip_ops(hip_ctx):
    from alpaca_amd.ops import HIPOps
    return HIPOps(hip_ctx)
