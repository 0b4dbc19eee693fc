"""Shared test setup: the `gpu` marker and import paths.

`-m "not gpu"` runs on any host (oracle pins, host logic, the C ABI's exports);
`-m gpu` runs the parity tests on an MI355X through the C ABI.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "lfm2-ampere_amd"), os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def oracle():
    import lk_oracle
    lk_oracle.load()
    return lk_oracle


@pytest.fixture(scope="session")
def lk():
    """The HIP library; GPU tests fail (not skip) if it is not built."""
    import torch
    import lk_attn
    assert torch.cuda.is_available(), "gpu tests need a GPU"
    lk_attn.load()
    return lk_attn


@pytest.fixture(scope="session")
def lk_host():
    """The HIP library for host-side entry points (no device needed)."""
    import lk_attn
    lk_attn.load()
    return lk_attn
