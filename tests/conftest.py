"""pytest configuration: the `gpu` marker and import paths.

`-m "not gpu"` runs the oracle, fixture, host-logic and C-ABI export tests
(no device needed); `-m gpu` runs the parity tests on an MI355X.
"""
import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_SRC = os.path.join(REPO, "flash-attention-sm75-register-fused_amd", "src")
for p in (REPO, PKG_SRC):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def device():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test requested but no HIP device is visible")
    return torch.device("cuda", 0)
