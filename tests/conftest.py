"""Test configuration: the `gpu` marker and import paths.

`-m "not gpu"` runs on any machine (oracle pins, host bookkeeping, ABI
exports); `-m gpu` needs an MI355X and calls the HIP library through its C ABI.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "lns-ml_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (gfx950) and the built liblnskv.so")


@pytest.fixture(scope="session")
def gpu():
    """Fails (does not skip) when a gpu-marked test runs without a GPU."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("gpu test run without a visible GPU")
    return torch.device("cuda", 0)
