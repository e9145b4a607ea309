"""Test configuration: the `gpu` marker and import paths.

CPU tests (`-m "not gpu"`) cover the oracle against golden vectors and closed forms, the
host-side logic, and that the C-ABI library loads and exports every declared symbol.
GPU tests (`-m gpu`) call the HIP library through its C ABI and compare with the oracle.
"""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("", "oracle", "ltx-2.5-swift_amd"):
    path = os.path.join(ROOT, sub)
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def device():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test collected on a host without a GPU (run with -m 'not gpu')")
    return torch.device("cuda:0")
