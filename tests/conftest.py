"""Shared pytest configuration.

Tests marked ``gpu`` run the HIP kernels on a real MI355X through the C ABI; the
rest (oracle pinning, host logic, C-ABI symbol/validation checks) run on the CPU.
"""

from __future__ import annotations

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libkore_amd.so")


@pytest.fixture(scope="session")
def gpu():
    """Fail loudly (never skip) when a gpu-marked test has no GPU or no library."""
    import torch

    assert torch.cuda.is_available(), "gpu-marked test needs a HIP device"
    import kore_amd._lib as L

    L.load()
    name = torch.cuda.get_device_properties(0).gcnArchName
    assert "gfx950" in name, f"expected gfx950, got {name}"
    return torch.device("cuda:0")
