"""Shared pytest configuration.

Markers:
  gpu  -- needs a real MI355X (HIP device); the CPU suite runs with -m "not gpu".
"""
import os
import sys
from pathlib import Path

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
