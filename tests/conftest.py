"""Shared pytest configuration.

Markers:
  gpu  -- needs a real MI355X (HIP device); the CPU suite runs with -m "not gpu".
"""
import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: test needs a real MI355X GPU (HIP)")


@pytest.fixture(scope="session")
def golden_dir() -> Path:
    return GOLDEN


@pytest.fixture(scope="session")
def ctx():
    """A HIP context on cuda:0 bound to torch's current stream."""
    import torch
    import undertow_amd as U

    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    c = U.Context(0)
    yield c
    c.synchronize()


def dev(a, dtype=None):
    """numpy -> torch tensor on cuda:0."""
    import torch

    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.to(dtype)
    return t.to("cuda:0")


def host(t) -> np.ndarray:
    import torch

    torch.cuda.synchronize()
    return t.detach().cpu().numpy()
