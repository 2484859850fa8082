"""Shared pytest setup: the `gpu` marker, import paths, and small helpers."""
import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "flash-kernel-engine_amd")
for p in (REPO, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP C ABI)")


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as o
    o.build()
    o.lib()
    return o


@pytest.fixture(scope="session")
def dev():
    """The GPU used by `gpu` tests; fails (does not skip) without one."""
    import torch
    assert torch.cuda.is_available(), "gpu test needs a visible MI355X"
    return torch.device("cuda:0")
