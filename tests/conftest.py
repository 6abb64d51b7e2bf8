"""Shared test setup: the ``gpu`` marker, import paths, and tiny models.

``-m "not gpu"`` runs the oracle, host-logic and library-loading tests on the
CPU; ``-m gpu`` runs the parity tests on an MI355X (they call the HIP library
through its C ABI and compare with the oracle and the golden vectors).
"""

import sys
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(Path(__file__).resolve().parent))

GPU = torch.cuda.is_available()


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X) and the built HIP library")
    config.addinivalue_line("markers", "slow: long-running")


DEFAULT_GPU_TIMEOUT = 600   # seconds per GPU test when no --timeout is given; the longest takes ~40 s


def pytest_collection_modifyitems(config, items):
    skip = pytest.mark.skip(reason="no GPU in this environment")
    # A GPU test that hangs inside a device call ends the run with its name and stack (pytest-timeout's
    # thread method) instead of holding the GPU until an outer limit kills everything.
    bound = (pytest.mark.timeout(DEFAULT_GPU_TIMEOUT, method="thread")
             if GPU and config.pluginmanager.hasplugin("timeout") and not config.getoption("timeout", None)
             else None)
    for item in items:
        if "gpu" in item.keywords and not GPU:
            item.add_marker(skip)
        elif "gpu" in item.keywords and bound is not None and item.get_closest_marker("timeout") is None:
            item.add_marker(bound)


def tiny_mlp(seed=0, din=48, hidden=193, dout=5, dtype=torch.float32, device="cpu"):
    """The reference suite's small model (reference tests/conftest.py:19-26)."""
    torch.manual_seed(seed)
    return torch.nn.Sequential(
        torch.nn.Linear(din, hidden),
        torch.nn.GELU(),
        torch.nn.LayerNorm(hidden),
        torch.nn.Linear(hidden, dout),
    ).to(device=device, dtype=dtype)


def max_param_diff(a, b):
    return max((x.float() - y.float()).abs().max().item() for x, y in zip(a.parameters(), b.parameters()))
