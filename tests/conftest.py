"""Shared pytest set-up: import paths, the `gpu` marker, seeded inputs."""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "qwen-fieldfare_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture
def rng():
    return np.random.default_rng(0x5157454E)


def gpu_available():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def hip():
    """The product library through its C ABI; GPU tests only. Fails (does not
    skip) when a GPU is present but the HIP library is missing."""
    if not gpu_available():
        pytest.skip("no GPU in this container")
    import qff
    return qff.lib()
