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


# Error figures of the native path per benchmark configuration, printed at
# the end of the session (so they appear in the tail of a -q run).
_PARITY_LINES: list[str] = []


def error_figures(actual, expected) -> dict:
    """max_abs = max |a - e|; max_rel = max |a - e| / max |e| (the largest
    error relative to the tensor's largest magnitude); rel_l2 = ||a - e|| /
    ||e||, all in FP64 on the CPU."""

    import torch

    a = torch.as_tensor(actual).detach().to(device="cpu", dtype=torch.float64)
    e = torch.as_tensor(expected).detach().to(device="cpu", dtype=torch.float64)
    diff = (a - e).abs()
    scale = e.abs().max().clamp_min(1e-300)
    return {
        "max_abs": float(diff.max()),
        "max_rel": float(diff.max() / scale),
        "rel_l2": float((a - e).norm() / e.norm().clamp_min(1e-300)),
    }


@pytest.fixture(scope="session")
def parity_report():
    """record(config, actual, fp32_reference, fp64_reference) stores the
    native output's error figures against the FP32 CPU oracle and its rel-L2
    error against the FP64 oracle; record_grads(config, {name: (actual,
    fp64)}) stores gradients' rel-L2 errors against FP64 autograd."""

    class _Report:
        @staticmethod
        def record(config: str, actual, fp32, fp64) -> dict:
            figures = error_figures(actual, fp32)
            figures["rel_l2_fp64"] = error_figures(actual, fp64)["rel_l2"]
            _PARITY_LINES.append(
                f"{config}: vs FP32 CPU max_abs {figures['max_abs']:.3e} max_rel {figures['max_rel']:.3e} "
                f"rel_l2 {figures['rel_l2']:.3e}; vs FP64 rel_l2 {figures['rel_l2_fp64']:.3e}"
            )
            return figures

        @staticmethod
        def record_grads(config: str, pairs: dict) -> dict:
            errors = {name: error_figures(a, e)["rel_l2"] for name, (a, e) in pairs.items()}
            _PARITY_LINES.append(
                f"{config}: grad rel_l2 vs FP64 " + " ".join(f"{k} {v:.2e}" for k, v in errors.items())
            )
            return errors

    return _Report()


def pytest_terminal_summary(terminalreporter, exitstatus, config) -> None:
    if _PARITY_LINES:
        terminalreporter.write_sep("-", "native path error figures per configuration")
        for line in _PARITY_LINES:
            terminalreporter.write_line(line)


@pytest.fixture(scope="session")
def native():
    """The loaded native boundary module (lsso_amd.ball.hip)."""

    import torch

    from lsso_amd.ball import hip

    assert torch.cuda.is_available(), "gpu tests need a ROCm device"
    hip.load()
    return hip
