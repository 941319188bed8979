"""The C-ABI library on the CPU: it loads without a GPU, exports every entry
point that include/lsso_hip.h declares, and validates shapes, sizes and
arguments on the host before any launch (reference csrc/ball/common.cuh:
194-269).  No compute call is made here."""

from __future__ import annotations

import ctypes
from pathlib import Path
import re

import pytest
import torch  # noqa: F401  (loads the HIP runtime the library links against)

from lsso_amd.ball import hip

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "lsso_hip.h"


def _declared_functions() -> set[str]:
    text = HEADER.read_text()
    return set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\*?(lsso_hip_\w+)\s*\(", text, re.MULTILINE))


@pytest.fixture(scope="module")
def library() -> ctypes.CDLL:
    path = hip.default_library_path()
    if not path.is_file():
        pytest.fail(f"the native library is not built at {path}; run __graft_entry__.build()")
    return hip.open_library(path)


def test_library_exports_every_declared_function(library) -> None:
    declared = _declared_functions()
    assert {"lsso_hip_mixer_forward", "lsso_hip_mixer_backward", "lsso_hip_linear"} <= declared
    for name in sorted(declared):
        assert hasattr(library, name), name
    assert set(hip._SYMBOLS) == declared


def test_contract_version_and_target(library) -> None:
    assert library.lsso_hip_contract_version() == hip._NATIVE_CONTRACT_VERSION
    assert library.lsso_hip_target().decode() == "gfx950"


def _shape(batch=2, length=33, heads=2, rank=32, head_dim=17):
    return hip.MixerShape(batch, length, heads, rank, head_dim)


def _message(library) -> str:
    return library.lsso_hip_last_error().decode()


@pytest.mark.parametrize("rank", (16, 32, 48, 64))
def test_valid_shapes_are_accepted(library, rank) -> None:
    shape = _shape(rank=rank)
    assert library.lsso_hip_mixer_validate(ctypes.byref(shape), 0) == 0
    size = ctypes.c_size_t()
    assert library.lsso_hip_mixer_workspace_bytes(ctypes.byref(shape), 2, ctypes.byref(size)) == 0
    assert size.value > 0 and size.value % 256 == 0


@pytest.mark.parametrize(
    ("fields", "code", "message"),
    [
        ({"rank": 24}, -2, "rank in {16, 32, 48, 64}"),
        ({"batch": 0}, -1, "B, N, and H must be positive"),
        ({"length": 0}, -1, "B, N, and H must be positive"),
        ({"heads": 0}, -1, "B, N, and H must be positive"),
        ({"head_dim": 0}, -1, "nonempty content channel"),
    ],
)
def test_invalid_shapes_are_rejected_with_messages(library, fields, code, message) -> None:
    shape = _shape(**fields)
    assert library.lsso_hip_mixer_validate(ctypes.byref(shape), 0) == code
    assert message in _message(library)


def test_positions_mode_is_checked(library) -> None:
    shape = _shape()
    assert library.lsso_hip_mixer_validate(ctypes.byref(shape), 3) == -1
    assert "positions_mode" in _message(library)


def test_null_output_pointers_are_rejected(library) -> None:
    shape = _shape()
    size = ctypes.c_size_t()
    assert library.lsso_hip_mixer_workspace_bytes(ctypes.byref(shape), 0, None) == -1
    assert library.lsso_hip_mixer_tape_floats(ctypes.byref(shape), None) == -1
    assert library.lsso_hip_mixer_tape_floats(None, ctypes.byref(size)) == -1
    assert "shape must not be NULL" in _message(library)


def test_tape_holds_compact_state_only(library) -> None:
    batch, length, heads, rank, head_dim = 3, 4096, 8, 48, 32
    shape = _shape(batch, length, heads, rank, head_dim)
    floats = ctypes.c_size_t()
    assert library.lsso_hip_mixer_tape_floats(ctypes.byref(shape), ctypes.byref(floats)) == 0
    assert floats.value == batch * heads * (4 * rank * rank + 2 * rank * head_dim)


def test_forward_rejects_missing_buffers_before_launch(library) -> None:
    shape = _shape()
    status = library.lsso_hip_mixer_forward(
        ctypes.byref(shape), None, None, None, None, None, None, 0, None, None, None, None, 0, None
    )
    assert status == -1
    assert "must not be NULL" in _message(library)


def test_forward_rejects_a_small_workspace(library) -> None:
    shape = _shape()
    fake = ctypes.c_void_p(1 << 20)  # never dereferenced: validation fails first
    status = library.lsso_hip_mixer_forward(
        ctypes.byref(shape), fake, fake, fake, fake, None, None, 0, None, fake, None, fake, 16, None
    )
    assert status == -1
    assert "workspace" in _message(library)


def test_fused_projection_envelope(library) -> None:
    assert library.lsso_hip_mixer_projected_supported(ctypes.byref(_shape(heads=8, rank=32, head_dim=32))) == 1
    assert library.lsso_hip_mixer_projected_supported(ctypes.byref(_shape(heads=2, rank=32, head_dim=96))) == 0
    assert library.lsso_hip_mixer_projected_supported(ctypes.byref(_shape(heads=9, rank=16, head_dim=16))) == 0
    # Packed rows up to 640 columns (rank 48 at H = 8, d = 32), not 768.
    assert library.lsso_hip_mixer_projected_supported(ctypes.byref(_shape(heads=8, rank=48, head_dim=32))) == 1
    assert library.lsso_hip_mixer_projected_supported(ctypes.byref(_shape(heads=8, rank=64, head_dim=32))) == 0
    assert library.lsso_hip_mixer_projected_supported(ctypes.byref(_shape(rank=20))) == -2


def test_backward_envelope_and_workspace(library) -> None:
    size = ctypes.c_size_t()
    shape = _shape(heads=8, rank=48, head_dim=32, length=2048, batch=4)
    assert library.lsso_hip_mixer_backward_workspace_bytes(ctypes.byref(shape), 0, ctypes.byref(size)) == 0
    assert size.value > 0
    # Any head_dim: wide heads run the panel-looped compact VJP.
    for head_dim in (65, 257, 512):
        wide = _shape(head_dim=head_dim)
        assert library.lsso_hip_mixer_backward_workspace_bytes(ctypes.byref(wide), 0, ctypes.byref(size)) == 0
        assert size.value > 0
    bad_rank = _shape(rank=24)
    assert library.lsso_hip_mixer_backward_workspace_bytes(ctypes.byref(bad_rank), 0, ctypes.byref(size)) == -2


def test_linear_validation(library) -> None:
    size = ctypes.c_size_t()
    assert library.lsso_hip_linear_workspace_bytes(10, 256, 512, ctypes.byref(size)) == 0
    assert size.value == 0
    assert library.lsso_hip_linear_workspace_bytes(-1, 256, 512, ctypes.byref(size)) == -1
    # Any in_features (past 640 the K-streaming tier): only arguments are checked.
    status = library.lsso_hip_linear(None, 1, 4, 700, 700, None, None, None, 8, None, 1, None, 0, None)
    assert status == -1
    assert "must not be NULL" in _message(library)
    status = library.lsso_hip_linear(None, 1, 4, 700, 600, None, None, None, 8, None, 1, None, 0, None)
    assert status == -1
    assert "x_row_stride" in _message(library)


def test_weight_gradient_validation(library) -> None:
    size = ctypes.c_size_t()
    assert library.lsso_hip_linear_weight_grad_workspace_bytes(131072, 256, 640, ctypes.byref(size)) == 0
    assert size.value >= 640 * 256 * 4 and size.value % 256 == 0
    assert library.lsso_hip_linear_weight_grad_workspace_bytes(0, 256, 640, ctypes.byref(size)) == 0
    # 1,024 output tiles fill every resident slot: one row split, so the
    # FP32 partials are one [N, K] block plus one bias row, not eight.
    assert library.lsso_hip_linear_weight_grad_workspace_bytes(131072, 4096, 4096, ctypes.byref(size)) == 0
    assert size.value == 4096 * 4096 * 4 + 4096 * 4
    assert library.lsso_hip_linear_weight_grad_workspace_bytes(-1, 256, 640, ctypes.byref(size)) == -1
    fake = ctypes.c_void_p(1 << 20)  # never dereferenced: validation fails first
    status = library.lsso_hip_linear_weight_grad(fake, 1, 64, fake, 3, 64, 10, 64, 64, None, fake, None,
                                                 fake, 1 << 20, None)
    assert status == -2 and "float16 or bfloat16" in _message(library)
    status = library.lsso_hip_linear_weight_grad(fake, 1, 32, fake, 1, 64, 10, 64, 64, None, fake, None,
                                                 fake, 1 << 20, None)
    assert status == -1 and "g_row_stride" in _message(library)
    status = library.lsso_hip_linear_weight_grad(fake, 1, 64, fake, 1, 64, 10, 64, 64, None, None, None,
                                                 fake, 1 << 20, None)
    assert status == -1 and "grad_weight" in _message(library)
    status = library.lsso_hip_linear_weight_grad(fake, 1, 64, fake, 1, 64, 10, 64, 64, None, fake, None,
                                                 fake, 16, None)
    assert status == -1 and "workspace" in _message(library)


def test_project_mix_forward_validates_before_launch(library) -> None:
    fake = ctypes.c_void_p(1 << 20)  # never dereferenced: validation fails first
    # head_dim 17 is outside the fused envelope (a multiple of 16 is needed).
    status = library.lsso_hip_project_mix_forward(
        ctypes.byref(_shape()), fake, 1, fake, None, None, fake, fake, fake, None, None, 0, None,
        fake, fake, None, fake, 1 << 30, None,
    )
    assert status == -2
    assert "lsso_hip_linear and lsso_hip_mixer_forward" in _message(library)
    shape = _shape(heads=8, rank=48, head_dim=32)
    status = library.lsso_hip_project_mix_forward(
        ctypes.byref(shape), fake, 3, fake, None, None, fake, fake, fake, None, None, 0, None,
        fake, fake, None, fake, 1 << 30, None,
    )
    assert status == -1
    assert "x_dtype" in _message(library)
    status = library.lsso_hip_project_mix_forward(
        ctypes.byref(shape), None, 1, fake, None, None, fake, fake, fake, None, None, 0, None,
        fake, fake, None, fake, 1 << 30, None,
    )
    assert status == -1
    assert "must not be NULL" in _message(library)
    status = library.lsso_hip_project_mix_forward(
        ctypes.byref(shape), fake, 1, fake, None, None, fake, fake, fake, None, None, 0, None,
        fake, fake, None, fake, 16, None,
    )
    assert status == -1
    assert "workspace" in _message(library)


def test_grad_columns_validation(library) -> None:
    size = ctypes.c_size_t()
    assert library.lsso_hip_linear_grad_columns_workspace_bytes(0, 256, ctypes.byref(size)) == 0
    assert size.value == 0
    assert library.lsso_hip_linear_grad_columns_workspace_bytes(131072, 640, ctypes.byref(size)) == 0
    assert size.value >= 640 * 4 and size.value % 256 == 0
    assert library.lsso_hip_linear_grad_columns_workspace_bytes(4, 0, ctypes.byref(size)) == -1
    status = library.lsso_hip_linear_grad_columns(None, 3, 4, 8, 8, None, None, None, None, 0, None)
    assert status == -2
    assert "float16 or bfloat16" in _message(library)
    status = library.lsso_hip_linear_grad_columns(None, 1, 4, 8, 4, None, None, None, None, 0, None)
    assert status == -1
    assert "g_row_stride" in _message(library)
    # Nothing asked for: no launch, no error.
    assert library.lsso_hip_linear_grad_columns(None, 1, 4, 8, 8, None, None, None, None, 0, None) == 0
    sums = ctypes.c_void_p(256)
    status = library.lsso_hip_linear_grad_columns(ctypes.c_void_p(512), 1, 4, 8, 8, None, None,
                                                  sums, None, 0, None)
    assert status == -1
    assert "workspace" in _message(library)


def test_errors_are_thread_local(library) -> None:
    import threading

    shape = _shape(rank=24)
    assert library.lsso_hip_mixer_validate(ctypes.byref(shape), 0) == -2
    seen = []

    def other() -> None:
        good = _shape()
        library.lsso_hip_mixer_validate(ctypes.byref(good), 0)
        seen.append(_message(library))

    thread = threading.Thread(target=other)
    thread.start()
    thread.join()
    assert seen == [""]
    assert "rank in" in _message(library)


def test_probe_library_rejects_sizes_before_launch() -> None:
    """The benchmark's HBM probes (liblsso_probe_gfx950.so, outside the
    mixer's C ABI) load without a GPU and refuse sizes that are not whole
    4,096-byte granules, and null or unaligned buffers, before any launch."""
    from lsso_amd.build import probe_library_path

    path = probe_library_path()
    if not path.is_file():
        pytest.fail(f"the probe library is not built at {path}; run __graft_entry__.build()")
    probe = ctypes.CDLL(str(path))
    probe.lsso_probe_copy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint64,
                                      ctypes.c_int, ctypes.c_void_p]
    probe.lsso_probe_read.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint64,
                                      ctypes.c_void_p]
    probe.lsso_probe_write.argtypes = [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p]
    aligned = 1 << 20
    assert probe.lsso_probe_copy(aligned, aligned, 0, 0, None) == 22
    assert probe.lsso_probe_copy(aligned, aligned, 4096 + 16, 0, None) == 22
    assert probe.lsso_probe_copy(aligned + 8, aligned, 4096, 1, None) == 22
    assert probe.lsso_probe_copy(None, aligned, 4096, 0, None) == 22
    assert probe.lsso_probe_read(aligned, None, 4096, None) == 22
    assert probe.lsso_probe_write(aligned, 100, None) == 22
    probe.lsso_probe_write_policy.argtypes = [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_int,
                                              ctypes.c_void_p]
    assert probe.lsso_probe_write_policy(aligned, 4096, 1, None) == 22
    assert probe.lsso_probe_write_policy(aligned, 100, 2, None) == 22
