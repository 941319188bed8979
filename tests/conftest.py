"""Shared test configuration.

``gpu`` tests need a gfx950 device and the in-tree native library; every
other test runs on CPU.  GPU tests load the library strictly: a missing or
stale library fails the test instead of skipping it.
"""

from __future__ import annotations

from pathlib import Path
import sys

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: requires an MI355X (gfx950) device and the native library")


@pytest.fixture(scope="session")
def native():
    """The loaded native boundary module (lsso_amd.ball.hip)."""

    import torch

    from lsso_amd.ball import hip

    assert torch.cuda.is_available(), "gpu tests need a ROCm device"
    hip.load()
    return hip
