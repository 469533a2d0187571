import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X) and the built library")


@pytest.fixture(scope="session")
def device():
    """The HIP device for `gpu` tests; fails (never skips) when there is none, so a GPU run
    cannot pass without exercising the kernels."""
    import torch
    if not torch.cuda.is_available():
        pytest.fail("gpu test selected but no HIP device is visible")
    from compactlogic_amd import _capi
    _capi.load()
    return torch.device("cuda:0")


def pytest_runtest_setup(item):
    # Name the case before it touches the GPU, so a fatal fault still shows which test ran.
    if item.get_closest_marker("gpu") is not None:
        print(f"\n[gpu-test] {item.nodeid}", flush=True)
