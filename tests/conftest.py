"""Test configuration: import paths and the `gpu` marker.

CPU tests (``-m "not gpu"``) cover the oracle against the reference's closed
forms and fixtures, the host-side argument checks, and that the C-ABI library
loads and exports every symbol ``include/hipenvs.h`` declares. GPU tests
(``-m gpu``) are the parity tests proper: they call the HIP kernels through
the C ABI and compare with the oracle on the same seeded inputs.
"""

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "metal-rl-envs_amd"
for p in (str(ROOT), str(PKG)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU and the built libhipenvs.so")


@pytest.fixture(scope="session")
def dev():
    """The GPU device for parity tests; fails (does not skip) without one."""
    import torch

    assert torch.cuda.is_available(), "GPU test run without a visible ROCm GPU"
    from hipenvs import _lib

    assert _lib.LIB_PATH.exists(), f"{_lib.LIB_PATH} not built"
    return torch.device("cuda", 0)
