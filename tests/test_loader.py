"""The loader's failure contract and the operator registration, on the CPU.

Mirrors the reference's loader tests (tests/cuda/test_fast_path.py:240-432):
a misnamed artifact, a stale contract version, a library built for another
target, the not-loaded error, the cached check of an explicit load and the
load lock, with the device query and the dlopen replaced by fakes so that no
GPU is needed.  The operator tests check the ``torch.ops.lsso_equilibrium``
schemas against the reference's (csrc/ball/binding.cpp:80-95) and run the
fake implementations and autograd guards on meta tensors.
"""

from __future__ import annotations

import ctypes
from pathlib import Path
from threading import Event, Thread
import time

import pytest
import torch
from torch.fx.experimental.proxy_tensor import make_fx

from lsso_amd.ball import hip, ops

# The reference's schemas as binding.cpp:80-95 writes them.
REFERENCE_SCHEMAS = {
    "contract_version": "lsso_equilibrium::contract_version() -> int",
    "forward_inference": (
        "lsso_equilibrium::forward_inference(Tensor projected, Tensor core_base_raw, "
        "Tensor core_drive_weight, Tensor eta_raw, Tensor? centered_positions=None, "
        "Tensor? valid_counts=None) -> Tensor"
    ),
    "forward_train": (
        "lsso_equilibrium::forward_train(Tensor projected, Tensor core_base_raw, "
        "Tensor core_drive_weight, Tensor eta_raw, Tensor? centered_positions=None, "
        "Tensor? valid_counts=None) -> (Tensor, Tensor, Tensor)"
    ),
    "backward": (
        "lsso_equilibrium::backward(Tensor grad_output, Tensor projected, Tensor core_base_raw, "
        "Tensor core_drive_weight, Tensor eta_raw, Tensor tape, Tensor pivots, "
        "Tensor? centered_positions=None, Tensor? valid_counts=None) -> (Tensor, Tensor, Tensor, Tensor)"
    ),
}


class FakeLibrary:
    """Stands in for the dlopened library: the two queries load() makes."""

    def __init__(self, version: int = hip._NATIVE_CONTRACT_VERSION, target: bytes = b"gfx950",
                 delay: float = 0.0) -> None:
        self.version = version
        self.target = target
        self.delay = delay

    def lsso_hip_contract_version(self) -> int:
        if self.delay:
            time.sleep(self.delay)
        return self.version

    def lsso_hip_target(self) -> bytes:
        return self.target


@pytest.fixture
def unloaded(monkeypatch: pytest.MonkeyPatch):
    """A process state with no library loaded and a gfx950 device."""

    monkeypatch.setattr(hip, "_LIBRARY", None)
    monkeypatch.setattr(hip, "_LOADED_ARCHITECTURE", None)
    monkeypatch.setattr(hip, "_device_architecture", lambda device=None: "gfx950")
    monkeypatch.setattr(ops, "register", lambda: None)
    return monkeypatch


def _artifact(tmp_path: Path, name: str = "liblsso_hip_gfx950.so") -> Path:
    library = tmp_path / name
    library.touch()
    return library


def test_default_library_path_is_target_specific(monkeypatch: pytest.MonkeyPatch) -> None:
    monkeypatch.delenv("LSSO_HIP_LIBRARY", raising=False)
    assert hip.default_library_path().name == "liblsso_hip_gfx950.so"
    monkeypatch.setenv("LSSO_HIP_LIBRARY", "/somewhere/liblsso_hip_gfx950.so")
    assert hip.default_library_path() == Path("/somewhere/liblsso_hip_gfx950.so")


def test_loader_rejects_a_misnamed_artifact(unloaded, tmp_path: Path) -> None:
    unloaded.setattr(hip, "open_library", lambda path=None: pytest.fail("must not dlopen"))
    with pytest.raises(RuntimeError, match="requires liblsso_hip_gfx950.so for gfx950, got lsso_equilibrium.so"):
        hip.load(path=_artifact(tmp_path, "lsso_equilibrium.so"))
    assert hip._LIBRARY is None and not hip.is_available()


def test_loader_rejects_a_missing_artifact(unloaded, tmp_path: Path) -> None:
    with pytest.raises(RuntimeError, match="was not found"):
        hip.load(path=tmp_path / "liblsso_hip_gfx950.so")


def test_loader_rejects_a_stale_same_name_artifact(unloaded, tmp_path: Path) -> None:
    library = _artifact(tmp_path)
    opened = []

    def open_library(path=None):
        opened.append(Path(path))
        return FakeLibrary(version=hip._NATIVE_CONTRACT_VERSION - 1)

    unloaded.setattr(hip, "open_library", open_library)
    with pytest.raises(RuntimeError, match="native contract version 0, but this package requires 1"):
        hip.load(path=library)
    assert opened == [library]
    assert hip._LIBRARY is None and hip._LOADED_ARCHITECTURE is None


def test_loader_rejects_a_library_for_another_target(unloaded, tmp_path: Path) -> None:
    unloaded.setattr(hip, "open_library", lambda path=None: FakeLibrary(target=b"gfx942"))
    with pytest.raises(RuntimeError, match="targets gfx942, not requested gfx950"):
        hip.load(path=_artifact(tmp_path))
    assert hip._LIBRARY is None


def test_device_architecture_requires_a_rocm_device(monkeypatch: pytest.MonkeyPatch) -> None:
    monkeypatch.setattr(hip.torch.cuda, "is_available", lambda: False)
    with pytest.raises(RuntimeError, match="requires an available ROCm device"):
        hip._device_architecture()


def test_device_architecture_rejects_other_targets(monkeypatch: pytest.MonkeyPatch) -> None:
    class Properties:
        gcnArchName = "gfx942:sramecc+:xnack-"

    monkeypatch.setattr(hip.torch.cuda, "is_available", lambda: True)
    monkeypatch.setattr(hip.torch.cuda, "current_device", lambda: 0)
    monkeypatch.setattr(hip.torch.cuda, "get_device_properties", lambda device: Properties())
    with pytest.raises(RuntimeError, match="supports gfx950 \\(MI355X\\); got gfx942"):
        hip._device_architecture()
    Properties.gcnArchName = "gfx950:sramecc+:xnack-"
    assert hip._device_architecture() == "gfx950"
    with pytest.raises(ValueError, match="requires a ROCm device, got cpu"):
        hip._device_architecture("cpu")


def test_not_loaded_is_an_error_everywhere(unloaded) -> None:
    message = "HIP extension is not loaded"
    with pytest.raises(RuntimeError, match=message):
        hip.require_available()
    projected = torch.zeros(1, 4, 48, dtype=torch.bfloat16)
    base, drive, eta = torch.zeros(2, 16, 16), torch.zeros(2, 8, 16), torch.zeros(2)
    with pytest.raises(RuntimeError, match=message):
        hip.fast_mix(projected, base, drive, eta)
    with pytest.raises(RuntimeError, match=message):
        hip.forward_inference(projected, base, drive, eta)
    with pytest.raises(RuntimeError, match=message):
        hip.linear(torch.zeros(1, 4, 8, dtype=torch.float16), torch.zeros(8, 8), None, torch.bfloat16)
    assert not hip.is_available()


def test_fast_mix_rejects_metadata_gradients_before_the_load_check(unloaded) -> None:
    projected = torch.zeros(1, 4, 48, dtype=torch.bfloat16)
    base, drive, eta = torch.zeros(2, 16, 16), torch.zeros(2, 8, 16), torch.zeros(2)
    with pytest.raises(ValueError, match="gradients for centered_positions"):
        hip.fast_mix(projected, base, drive, eta, torch.zeros(4, requires_grad=True))
    with pytest.raises(ValueError, match="gradients for valid_counts"):
        hip.fast_mix(projected, base, drive, eta, None, torch.ones(1, requires_grad=True))


def test_require_available_caches_a_verified_load(unloaded, tmp_path: Path) -> None:
    unloaded.setattr(hip, "open_library", lambda path=None: FakeLibrary())
    hip.load(path=_artifact(tmp_path))
    assert hip._LOADED_ARCHITECTURE == "gfx950"
    # The cached check does not query the library or the lock again.
    unloaded.setattr(hip, "_native_contract_version", lambda library: pytest.fail("queried again"))
    hip.require_available()
    # A second load is a no-op once a library is loaded.
    unloaded.setattr(hip, "open_library", lambda path=None: pytest.fail("dlopened twice"))
    hip.load(path=_artifact(tmp_path))


def test_loader_rejects_a_different_loaded_target(unloaded) -> None:
    unloaded.setattr(hip, "_LIBRARY", FakeLibrary())
    unloaded.setattr(hip, "_LOADED_ARCHITECTURE", "gfx942")
    with pytest.raises(RuntimeError, match="targets gfx942, not requested gfx950"):
        hip.load()


def test_concurrent_loads_open_the_library_once(unloaded, tmp_path: Path) -> None:
    library = _artifact(tmp_path)
    opened = []

    def open_library(path=None):
        opened.append(path)
        return FakeLibrary(delay=0.05)

    unloaded.setattr(hip, "open_library", open_library)
    errors: list[BaseException] = []

    def worker() -> None:
        try:
            hip.load(path=library)
        except BaseException as error:  # noqa: BLE001 - reported below
            errors.append(error)

    threads = [Thread(target=worker) for _ in range(8)]
    for thread in threads:
        thread.start()
    for thread in threads:
        thread.join(timeout=10.0)
    assert not errors
    assert len(opened) == 1
    assert hip._LOADED_ARCHITECTURE == "gfx950"


def test_loader_serializes_a_mixed_target_race(unloaded) -> None:
    """A load waiting on the lock sees the target that the holder loaded."""

    started, finished = Event(), Event()
    errors: list[RuntimeError] = []

    def request() -> None:
        started.set()
        try:
            hip.load()
        except RuntimeError as error:
            errors.append(error)
        finally:
            finished.set()

    with hip._LOAD_LOCK:
        thread = Thread(target=request)
        thread.start()
        assert started.wait(timeout=1.0)
        assert not finished.wait(timeout=0.1)
        unloaded.setattr(hip, "_LIBRARY", FakeLibrary())
        unloaded.setattr(hip, "_LOADED_ARCHITECTURE", "gfx942")
    thread.join(timeout=2.0)
    assert finished.is_set()
    assert len(errors) == 1 and "targets gfx942, not requested gfx950" in str(errors[0])


# --- torch.ops.lsso_equilibrium -------------------------------------------


@pytest.fixture(scope="module")
def registered():
    ops.register()
    ops.register()  # idempotent
    return torch.ops.lsso_equilibrium


def test_operator_schemas_are_the_reference_schemas(registered) -> None:
    for name, schema in REFERENCE_SCHEMAS.items():
        assert str(getattr(registered, name).default._schema) == schema


def _meta_inputs(batch=2, length=5, heads=3, rank=16, head_dim=8):
    projected = torch.empty(batch, length, heads * (rank + head_dim), dtype=torch.bfloat16, device="meta")
    base = torch.empty(heads, rank, rank, device="meta")
    drive = torch.empty(heads, head_dim, rank, device="meta")
    eta = torch.empty(heads, device="meta")
    return projected, base, drive, eta


@pytest.mark.parametrize("rank, head_dim", [(16, 8), (32, 32), (48, 17), (64, 64)])
def test_fake_implementations_give_the_library_shapes(registered, rank, head_dim) -> None:
    projected, base, drive, eta = _meta_inputs(rank=rank, head_dim=head_dim)
    output = registered.forward_inference(projected, base, drive, eta)
    assert output.shape == (2, 5, 3 * head_dim) and output.dtype == torch.bfloat16
    output, tape, pivots = registered.forward_train(projected, base, drive, eta)
    assert output.shape == (2, 5, 3 * head_dim)
    assert pivots.shape == (0,) and pivots.dtype == torch.int32
    path = hip.default_library_path()
    if path.is_file():
        library = hip.open_library(path)
        floats = ctypes.c_size_t()
        shape = hip.MixerShape(2, 5, 3, rank, head_dim)
        assert library.lsso_hip_mixer_tape_floats(ctypes.byref(shape), ctypes.byref(floats)) == 0
        assert tape.shape == (floats.value,) and tape.dtype == torch.float32
    grads = registered.backward(output, projected, base, drive, eta, tape, pivots)
    assert [g.shape for g in grads] == [projected.shape, base.shape, drive.shape, eta.shape]


def test_forward_operators_reject_autograd(registered) -> None:
    projected, base, drive, eta = _meta_inputs()
    base.requires_grad_(True)
    with pytest.raises(RuntimeError, match="forward_inference is an inference-only entry point"):
        registered.forward_inference(projected, base, drive, eta)
    with pytest.raises(RuntimeError, match="forward_train is a private tape-producing entry point"):
        registered.forward_train(projected, base, drive, eta)
    with torch.no_grad():
        assert registered.forward_inference(projected, base, drive, eta).shape == (2, 5, 24)


def test_operators_trace_without_a_graph_break(registered) -> None:
    def mix(projected, base, drive, eta):
        output, tape, pivots = registered.forward_train(projected, base, drive, eta)
        grads = registered.backward(output, projected, base, drive, eta, tape, pivots)
        return registered.forward_inference(projected, base, drive, eta), grads[0]

    graph = make_fx(mix, tracing_mode="fake")(*_meta_inputs())
    targets = [str(node.target) for node in graph.graph.nodes
               if isinstance(node.target, torch._ops.OpOverload)]
    assert targets == [
        "lsso_equilibrium.forward_train.default",
        "lsso_equilibrium.backward.default",
        "lsso_equilibrium.forward_inference.default",
    ]
