import os
import sys

import pytest

try:  # one HIP runtime per process: torch's copy, loaded before libvla_simd_hip.so
    import torch  # noqa: F401
except ImportError:
    pass

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU and the built libvla_simd_hip.so")


@pytest.fixture(scope="session")
def vla():
    """The HIP backend. A GPU test that gets here without a usable device fails
    (there is no CPU fallback to pass on)."""
    from helpers import load_pkg

    pkg = load_pkg()
    pkg.lib()
    assert pkg.int8_available(), "no gfx950 device visible to libvla_simd_hip.so"
    print("device:", pkg.device_name(), flush=True)
    return pkg


@pytest.fixture(scope="session")
def orc():
    from helpers import oracle

    return oracle()


@pytest.fixture(scope="session")
def torch_cuda():
    import torch

    assert torch.cuda.is_available(), "torch sees no GPU"
    return torch
