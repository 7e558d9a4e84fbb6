import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
PKG = ROOT / "ernie-image-ncnn-vulkan_amd"
for p in (ROOT / "oracle", PKG, ROOT / "tests"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) HIP device")
    config.addinivalue_line("markers", "slow: full-size case (seconds of device and host work)")


@pytest.fixture(scope="session")
def torch_mod():
    import torch
    return torch


@pytest.fixture(scope="session")
def ctx():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test collected without a HIP device")
    import ernie_amd
    c = ernie_amd.Context(0)
    yield c
    c.close()
