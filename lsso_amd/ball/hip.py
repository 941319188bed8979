"""Strict loader and PyTorch boundary of the gfx950 native library.

Mirrors the reference's native boundary ``lsso.ball.cuda``
(lsso/ball/cuda.py:57-326): an explicit ``load()``, ``is_available()``,
``require_available()`` and ``fast_mix()`` with train/inference selection,
plus the biased projection that replaces the reference's Triton GEMM
(lsso/ball/reference.py:20-75).  The library is the C ABI declared in
``include/lsso_hip.h``; PyTorch only supplies device memory and the current
stream.  There is no fallback: every entry point raises when the library is
not loaded or an input is outside the native contract.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path
from threading import Lock

import torch

from . import ops
from .reference import rotary_inverse_frequency

_LOAD_LOCK = Lock()
_NATIVE_CONTRACT_VERSION = 1
_SUPPORTED_ARCHITECTURES = frozenset(("gfx950",))
_LOADED_ARCHITECTURE: str | None = None
_LIBRARY: ctypes.CDLL | None = None
_INVERSE_FREQUENCY: dict[int, ctypes.Array] = {}

_F16 = 1
_BF16 = 2
_POSITIONS_DEFAULT = 0
_POSITIONS_SHARED = 1
_POSITIONS_BATCHED = 2

_SYMBOLS = (
    "lsso_hip_contract_version",
    "lsso_hip_target",
    "lsso_hip_last_error",
    "lsso_hip_mixer_validate",
    "lsso_hip_mixer_workspace_bytes",
    "lsso_hip_mixer_tape_floats",
    "lsso_hip_mixer_forward",
    "lsso_hip_mixer_forward_static",
    "lsso_hip_mixer_projected_supported",
    "lsso_hip_mixer_forward_projected",
    "lsso_hip_mixer_backward_workspace_bytes",
    "lsso_hip_mixer_backward",
    "lsso_hip_mixer_backward_ex",
    "lsso_hip_linear_workspace_bytes",
    "lsso_hip_linear",
    "lsso_hip_linear_grad_columns_workspace_bytes",
    "lsso_hip_linear_grad_columns",
    "lsso_hip_layer_supported",
    "lsso_hip_layer_workspace_bytes",
    "lsso_hip_layer_forward",
    "lsso_hip_layer_forward_timed",
    "lsso_hip_project_mix_forward",
    "lsso_hip_layer_forward_train",
    "lsso_hip_linear_weight_grad_workspace_bytes",
    "lsso_hip_linear_weight_grad",
)


class MixerShape(ctypes.Structure):
    """``lsso_hip_mixer_shape`` (include/lsso_hip.h)."""

    _fields_ = [
        ("batch", ctypes.c_int64),
        ("length", ctypes.c_int64),
        ("heads", ctypes.c_int64),
        ("rank", ctypes.c_int64),
        ("head_dim", ctypes.c_int64),
    ]


def _declare(library: ctypes.CDLL) -> None:
    vp = ctypes.c_void_p
    i64 = ctypes.c_int64
    shape_p = ctypes.POINTER(MixerShape)
    size_p = ctypes.POINTER(ctypes.c_size_t)
    library.lsso_hip_contract_version.restype = ctypes.c_int
    library.lsso_hip_contract_version.argtypes = []
    library.lsso_hip_target.restype = ctypes.c_char_p
    library.lsso_hip_target.argtypes = []
    library.lsso_hip_last_error.restype = ctypes.c_char_p
    library.lsso_hip_last_error.argtypes = []
    library.lsso_hip_mixer_validate.restype = ctypes.c_int
    library.lsso_hip_mixer_validate.argtypes = [shape_p, ctypes.c_int]
    library.lsso_hip_mixer_workspace_bytes.restype = ctypes.c_int
    library.lsso_hip_mixer_workspace_bytes.argtypes = [shape_p, ctypes.c_int, size_p]
    library.lsso_hip_mixer_tape_floats.restype = ctypes.c_int
    library.lsso_hip_mixer_tape_floats.argtypes = [shape_p, size_p]
    library.lsso_hip_mixer_forward.restype = ctypes.c_int
    library.lsso_hip_mixer_forward.argtypes = [
        shape_p, vp, vp, vp, vp, vp, vp, ctypes.c_int, vp, vp, vp, vp, ctypes.c_size_t, vp,
    ]
    library.lsso_hip_mixer_forward_static.restype = ctypes.c_int
    library.lsso_hip_mixer_forward_static.argtypes = [
        shape_p, vp, vp, vp, vp, vp, vp, ctypes.c_int, vp, vp, vp, vp,
    ]  # shape, projected, base, drive, eta, inv_freq, positions, mode, counts, output, tape, stream
    library.lsso_hip_mixer_projected_supported.restype = ctypes.c_int
    library.lsso_hip_mixer_projected_supported.argtypes = [shape_p]
    library.lsso_hip_mixer_forward_projected.restype = ctypes.c_int
    library.lsso_hip_mixer_forward_projected.argtypes = [
        shape_p, vp, vp, vp, vp, vp, vp, ctypes.c_int, vp, vp, vp, vp, vp, ctypes.c_int, vp,
        ctypes.c_size_t, vp,
    ]  # shape, projected, base, drive, eta, inv_freq, positions, mode, counts,
    #    out_weight, out_bias, row_mask, y, y_dtype, workspace, workspace_bytes, stream
    library.lsso_hip_mixer_backward_workspace_bytes.restype = ctypes.c_int
    library.lsso_hip_mixer_backward_workspace_bytes.argtypes = [shape_p, ctypes.c_int, size_p]
    library.lsso_hip_mixer_backward.restype = ctypes.c_int
    library.lsso_hip_mixer_backward.argtypes = [
        shape_p, vp, vp, vp, vp, vp, vp, vp, ctypes.c_int, vp, vp, vp, vp, vp, vp, vp,
        ctypes.c_size_t, vp,
    ]  # shape, grad_output, projected, base, drive, eta, inv_freq, positions, mode, counts,
    #    tape, grad_projected, grad_base, grad_drive, grad_eta, workspace, workspace_bytes, stream
    library.lsso_hip_mixer_backward_ex.restype = ctypes.c_int
    library.lsso_hip_mixer_backward_ex.argtypes = [
        shape_p, vp, vp, vp, vp, vp, vp, vp, ctypes.c_int, vp, vp, vp, vp, vp, vp, vp, vp,
        ctypes.c_size_t, vp,
    ]  # ... as lsso_hip_mixer_backward, with grad_projected_column_sums before the workspace
    library.lsso_hip_linear_workspace_bytes.restype = ctypes.c_int
    library.lsso_hip_linear_workspace_bytes.argtypes = [i64, i64, i64, size_p]
    library.lsso_hip_linear.restype = ctypes.c_int
    library.lsso_hip_linear.argtypes = [
        vp, ctypes.c_int, i64, i64, i64, vp, vp, vp, i64, vp, ctypes.c_int, vp, ctypes.c_size_t, vp,
    ]  # x, x_dtype, rows, in, stride, weight, bias, row_mask, out, y, y_dtype, ws, ws_bytes, stream
    library.lsso_hip_linear_grad_columns_workspace_bytes.restype = ctypes.c_int
    library.lsso_hip_linear_grad_columns_workspace_bytes.argtypes = [i64, i64, size_p]
    library.lsso_hip_linear_grad_columns.restype = ctypes.c_int
    library.lsso_hip_linear_grad_columns.argtypes = [
        vp, ctypes.c_int, i64, i64, i64, vp, vp, vp, vp, ctypes.c_size_t, vp,
    ]  # g, g_dtype, rows, cols, stride, row_mask, g_bf16, column_sums, ws, ws_bytes, stream
    library.lsso_hip_linear_weight_grad_workspace_bytes.restype = ctypes.c_int
    library.lsso_hip_linear_weight_grad_workspace_bytes.argtypes = [i64, i64, i64, size_p]
    library.lsso_hip_linear_weight_grad.restype = ctypes.c_int
    library.lsso_hip_linear_weight_grad.argtypes = [
        vp, ctypes.c_int, i64, vp, ctypes.c_int, i64, i64, i64, i64, vp, vp, vp, vp, ctypes.c_size_t, vp,
    ]  # g, g_dtype, g_stride, x, x_dtype, x_stride, rows, in, out, row_mask, grad_weight, grad_bias,
    #    ws, ws_bytes, stream
    library.lsso_hip_layer_supported.restype = ctypes.c_int
    library.lsso_hip_layer_supported.argtypes = [shape_p]
    library.lsso_hip_layer_workspace_bytes.restype = ctypes.c_int
    library.lsso_hip_layer_workspace_bytes.argtypes = [shape_p, ctypes.c_int, size_p]
    library.lsso_hip_layer_forward.restype = ctypes.c_int
    library.lsso_hip_layer_forward.argtypes = [
        shape_p, vp, ctypes.c_int, vp, vp, vp, vp, vp, vp, vp, vp, ctypes.c_int, vp, vp, vp, vp,
        ctypes.c_int, vp, ctypes.c_size_t, vp,
    ]  # shape, x, x_dtype, in_weight, in_bias, row_mask, base, drive, eta, inv_freq, positions,
    #    mode, counts, out_weight, out_bias, y, y_dtype, workspace, workspace_bytes, stream
    library.lsso_hip_layer_forward_timed.restype = ctypes.c_int
    library.lsso_hip_layer_forward_timed.argtypes = [
        *library.lsso_hip_layer_forward.argtypes, ctypes.POINTER(ctypes.c_void_p),
    ]  # ... as lsso_hip_layer_forward, then hipEvent_t events[8]


    library.lsso_hip_project_mix_forward.restype = ctypes.c_int
    library.lsso_hip_project_mix_forward.argtypes = [
        shape_p, vp, ctypes.c_int, vp, vp, vp, vp, vp, vp, vp, vp, ctypes.c_int, vp, vp, vp, vp, vp,
        ctypes.c_size_t, vp,
    ]  # shape, x, x_dtype, in_weight, in_bias, row_mask, base, drive, eta, inv_freq, positions,
    #    mode, counts, packed, mixed, tape, workspace, workspace_bytes, stream
    library.lsso_hip_layer_forward_train.restype = ctypes.c_int
    library.lsso_hip_layer_forward_train.argtypes = [
        shape_p, vp, ctypes.c_int, vp, vp, vp, vp, vp, vp, vp, vp, ctypes.c_int, vp, vp, vp, vp, vp, vp,
        vp, ctypes.c_int, vp, ctypes.c_size_t, vp,
    ]  # shape, x, x_dtype, in_weight, in_bias, row_mask, base, drive, eta, inv_freq, positions,
    #    mode, counts, out_weight, out_bias, packed, mixed, tape, y, y_dtype, workspace,
    #    workspace_bytes, stream


def default_library_path() -> Path:
    """``LSSO_HIP_LIBRARY`` or the in-tree build (reference cuda.py:165-175)."""

    override = os.environ.get("LSSO_HIP_LIBRARY")
    if override:
        return Path(override).expanduser()
    return Path(__file__).resolve().parents[1] / "_lib" / "liblsso_hip_gfx950.so"


def open_library(path: str | os.PathLike[str] | None = None) -> ctypes.CDLL:
    """dlopen the library and declare its C ABI without touching a GPU.

    PyTorch is imported first so that the HIP runtime it carries (same
    SONAME) serves the library as well.
    """

    library_path = Path(path) if path is not None else default_library_path()
    if not library_path.is_file():
        raise RuntimeError(
            f"the LSSO HIP library was not found at {library_path}; build it with "
            "`python -m lsso_amd.build` or pass its path to load()"
        )
    library = ctypes.CDLL(str(library_path.resolve()))
    _declare(library)
    return library


def _native_contract_version(library: ctypes.CDLL | None) -> int | None:
    if library is None:
        return None
    return int(library.lsso_hip_contract_version())


def is_available() -> bool:
    """Whether the strict DYNAMIC + Rank-Rotary library is loaded and its
    operators are registered under ``torch.ops.lsso_equilibrium`` (cuda.py:57-63)."""

    return (
        _LIBRARY is not None
        and _native_contract_version(_LIBRARY) == _NATIVE_CONTRACT_VERSION
        and ops.is_registered()
    )


def require_available() -> None:
    """Reject a native request until the library is loaded (cuda.py:66-80)."""

    if _LOADED_ARCHITECTURE is not None:
        return
    with _LOAD_LOCK:
        if _LOADED_ARCHITECTURE is not None:
            return
        raise RuntimeError(
            "the LSSO accretive-equilibrium HIP extension is not loaded; build it with "
            "`python -m lsso_amd.build`, then call lsso_amd.ball.hip.load(); "
            f"native contract version {_NATIVE_CONTRACT_VERSION} is required"
        )


def _device_architecture(device: torch.device | int | None = None) -> str:
    """gfx target of the requested device (cuda.py:83-110)."""

    if not torch.cuda.is_available():
        raise RuntimeError("the LSSO HIP fast path requires an available ROCm device")
    if device is None:
        resolved = torch.device("cuda", torch.cuda.current_device())
    elif isinstance(device, int):
        resolved = torch.device("cuda", device)
    else:
        resolved = torch.device(device)
    if resolved.type != "cuda":
        raise ValueError(f"the LSSO HIP fast path requires a ROCm device, got {resolved}")
    if resolved.index is None:
        resolved = torch.device("cuda", torch.cuda.current_device())
    name = str(getattr(torch.cuda.get_device_properties(resolved), "gcnArchName", ""))
    architecture = name.split(":")[0]
    if architecture not in _SUPPORTED_ARCHITECTURES:
        raise RuntimeError(
            f"the LSSO HIP fast path supports gfx950 (MI355X); got {architecture or 'unknown'}"
        )
    return architecture


def load(path: str | os.PathLike[str] | None = None, *, device: torch.device | int | None = None) -> None:
    """Load the one strict gfx950 library for this process (cuda.py:178-217)."""

    global _LIBRARY, _LOADED_ARCHITECTURE
    requested = _device_architecture(device)
    with _LOAD_LOCK:
        if _LIBRARY is not None:
            if _LOADED_ARCHITECTURE is not None and _LOADED_ARCHITECTURE != requested:
                raise RuntimeError(
                    f"the loaded LSSO HIP library targets {_LOADED_ARCHITECTURE}, "
                    f"not requested {requested}"
                )
            return
        library_path = Path(path) if path is not None else default_library_path()
        expected = f"liblsso_hip_{requested}.so"
        if library_path.name != expected:
            raise RuntimeError(
                f"the strict LSSO HIP fast path requires {expected} for {requested}, "
                f"got {library_path.name}"
            )
        library = open_library(library_path)
        version = _native_contract_version(library)
        if version != _NATIVE_CONTRACT_VERSION:
            raise RuntimeError(
                f"the LSSO HIP library has native contract version {version}, but this "
                f"package requires {_NATIVE_CONTRACT_VERSION}; rebuild it with "
                "`python -m lsso_amd.build` and restart the process"
            )
        target = library.lsso_hip_target().decode()
        if target != requested:
            raise RuntimeError(f"the LSSO HIP library targets {target}, not requested {requested}")
        _LIBRARY = library
        # The reference's operators appear under torch.ops.lsso_equilibrium
        # when its extension loads (binding.cpp:79-107); these are the same
        # schemas, backed by this library.
        ops.register()
        _LOADED_ARCHITECTURE = requested


def _library() -> ctypes.CDLL:
    require_available()
    assert _LIBRARY is not None
    return _LIBRARY


def _check(status: int, library: ctypes.CDLL) -> None:
    if status != 0:
        message = library.lsso_hip_last_error().decode()
        if status == -2:
            raise ValueError(message)
        raise RuntimeError(message)


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _inverse_frequency(rank: int) -> ctypes.Array:
    """Host FP32 frequencies computed exactly as the reference does (reference.py:704-707)."""

    cached = _INVERSE_FREQUENCY.get(rank)
    if cached is None:
        values = rotary_inverse_frequency(rank, torch.float32).tolist()
        cached = (ctypes.c_float * len(values))(*values)
        _INVERSE_FREQUENCY[rank] = cached
    return cached


def _require_device_tensor(value: torch.Tensor, name: str, device: torch.device) -> None:
    if value.device.type != "cuda":
        raise RuntimeError(f"{name} must be a CUDA (ROCm device) tensor")
    if value.device != device:
        raise RuntimeError(f"{name} must share projected.device() (got {value.device} vs {device})")


def _validate_mixer(
    projected: torch.Tensor,
    core_base_raw: torch.Tensor,
    core_drive_weight: torch.Tensor,
    eta_raw: torch.Tensor,
    centered_positions: torch.Tensor | None,
    valid_counts: torch.Tensor | None,
) -> tuple[MixerShape, int]:
    """Tensor-level checks of the native contract (csrc/ball/common.cuh:194-269)."""

    if projected.device.type != "cuda":
        raise RuntimeError("projected must be a CUDA (ROCm device) tensor")
    if projected.dim() != 3:
        raise RuntimeError(f"projected must have shape [B, N, H*R + D], got {tuple(projected.shape)}")
    if not projected.is_contiguous():
        raise RuntimeError("projected must be contiguous [B, N, H*R + D]")
    if projected.dtype != torch.bfloat16:
        raise RuntimeError(
            "projected must use bfloat16 under the mixed precision HIP contract, "
            f"got {projected.dtype}"
        )
    batch, length, width = projected.shape
    return _validate_core(
        projected.device, batch, length, width, core_base_raw, core_drive_weight, eta_raw,
        centered_positions, valid_counts,
    )


def _validate_core(
    device: torch.device,
    batch: int,
    length: int,
    width: int,
    core_base_raw: torch.Tensor,
    core_drive_weight: torch.Tensor,
    eta_raw: torch.Tensor,
    centered_positions: torch.Tensor | None,
    valid_counts: torch.Tensor | None,
) -> tuple[MixerShape, int]:
    """Checks of the compact parameters, positions and counts for a packed
    width of ``width`` columns (csrc/ball/common.cuh:194-269)."""

    for name, value in (
        ("core_base_raw", core_base_raw),
        ("core_drive_weight", core_drive_weight),
        ("eta_raw", eta_raw),
    ):
        if not value.is_contiguous():
            raise RuntimeError(f"{name} must be contiguous")
        _require_device_tensor(value, name, device)
        if value.dtype != torch.float32:
            raise RuntimeError(f"{name} must use float32")
    if core_base_raw.dim() != 3 or core_base_raw.shape[1] != core_base_raw.shape[2]:
        raise RuntimeError(f"core_base_raw must have shape [H, R, R], got {tuple(core_base_raw.shape)}")
    heads, rank = core_base_raw.shape[0], core_base_raw.shape[1]
    if batch <= 0 or length <= 0 or heads <= 0:
        raise RuntimeError("B, N, and H must be positive")
    if rank not in (16, 32, 48, 64):
        raise RuntimeError(f"the HIP fast path supports rank in {{16, 32, 48, 64}}, got {rank}")
    if width <= heads * rank:
        raise RuntimeError("projected width must exceed H*R for a nonempty content channel")
    dim = width - heads * rank
    if dim % heads:
        raise RuntimeError("projected content width D must be divisible by H")
    head_dim = dim // heads
    if tuple(core_drive_weight.shape) != (heads, head_dim, rank):
        raise RuntimeError(
            f"core_drive_weight must have shape [H, D/H, R], got {tuple(core_drive_weight.shape)}"
        )
    if tuple(eta_raw.shape) != (heads,):
        raise RuntimeError(f"eta_raw must have shape [H], got {tuple(eta_raw.shape)}")
    mode = _POSITIONS_DEFAULT
    if centered_positions is not None:
        _require_device_tensor(centered_positions, "centered_positions", device)
        if not centered_positions.is_contiguous():
            raise RuntimeError("centered_positions must be contiguous")
        if centered_positions.dtype != torch.float32:
            raise RuntimeError("centered_positions must use float32")
        if centered_positions.dim() == 1 and centered_positions.shape[0] == length:
            mode = _POSITIONS_SHARED
        elif centered_positions.dim() == 2 and tuple(centered_positions.shape) == (batch, length):
            mode = _POSITIONS_BATCHED
        else:
            raise RuntimeError(
                f"centered_positions must have shape [N] or [B, N], got {tuple(centered_positions.shape)}"
            )
    if valid_counts is not None:
        _require_device_tensor(valid_counts, "valid_counts", device)
        if not valid_counts.is_contiguous():
            raise RuntimeError("valid_counts must be contiguous")
        if valid_counts.dtype != torch.float32:
            raise RuntimeError("valid_counts must use float32")
        if valid_counts.dim() != 1 or valid_counts.shape[0] != batch:
            raise RuntimeError(f"valid_counts must have shape [B], got {tuple(valid_counts.shape)}")
    return MixerShape(batch, length, heads, rank, head_dim), mode


def _mixer_forward(
    projected: torch.Tensor,
    core_base_raw: torch.Tensor,
    core_drive_weight: torch.Tensor,
    eta_raw: torch.Tensor,
    centered_positions: torch.Tensor | None,
    valid_counts: torch.Tensor | None,
    record_tape: bool,
) -> tuple[torch.Tensor, torch.Tensor | None]:
    library = _library()
    shape, mode = _validate_mixer(
        projected, core_base_raw, core_drive_weight, eta_raw, centered_positions, valid_counts
    )
    device = projected.device
    workspace_bytes = ctypes.c_size_t()
    _check(library.lsso_hip_mixer_workspace_bytes(ctypes.byref(shape), mode, ctypes.byref(workspace_bytes)), library)
    output = torch.empty(
        (shape.batch, shape.length, shape.heads * shape.head_dim), dtype=torch.bfloat16, device=device
    )
    workspace = torch.empty(workspace_bytes.value, dtype=torch.uint8, device=device)
    tape = None
    if record_tape:
        floats = ctypes.c_size_t()
        _check(library.lsso_hip_mixer_tape_floats(ctypes.byref(shape), ctypes.byref(floats)), library)
        tape = torch.empty(floats.value, dtype=torch.float32, device=device)
    with torch.cuda.device(device):
        status = library.lsso_hip_mixer_forward(
            ctypes.byref(shape),
            projected.data_ptr(),
            core_base_raw.data_ptr(),
            core_drive_weight.data_ptr(),
            eta_raw.data_ptr(),
            ctypes.cast(_inverse_frequency(shape.rank), ctypes.c_void_p),
            None if centered_positions is None else centered_positions.data_ptr(),
            mode,
            None if valid_counts is None else valid_counts.data_ptr(),
            output.data_ptr(),
            None if tape is None else tape.data_ptr(),
            workspace.data_ptr(),
            workspace_bytes.value,
            _stream(device),
        )
    _check(status, library)
    return output, tape


def _any_requires_grad(*values: torch.Tensor | None) -> bool:
    return any(value is not None and value.requires_grad for value in values)


def forward_inference(
    projected: torch.Tensor,
    core_base_raw: torch.Tensor,
    core_drive_weight: torch.Tensor,
    eta_raw: torch.Tensor,
    centered_positions: torch.Tensor | None = None,
    valid_counts: torch.Tensor | None = None,
) -> torch.Tensor:
    """Inference-only native mixer (csrc/ball/binding.cpp:16-42)."""

    if torch.is_grad_enabled() and _any_requires_grad(
        projected, core_base_raw, core_drive_weight, eta_raw, centered_positions, valid_counts
    ):
        raise RuntimeError(
            "lsso_hip forward_inference is an inference-only entry point and cannot "
            "participate in autograd directly; use lsso_amd.ball.hip.fast_mix()"
        )
    output, _tape = _mixer_forward(
        projected, core_base_raw, core_drive_weight, eta_raw, centered_positions, valid_counts, False
    )
    return output


def forward_train(
    projected: torch.Tensor,
    core_base_raw: torch.Tensor,
    core_drive_weight: torch.Tensor,
    eta_raw: torch.Tensor,
    centered_positions: torch.Tensor | None = None,
    valid_counts: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Tape-producing native mixer (csrc/ball/binding.cpp:44-70)."""

    if torch.is_grad_enabled() and _any_requires_grad(
        projected, core_base_raw, core_drive_weight, eta_raw, centered_positions, valid_counts
    ):
        raise RuntimeError(
            "lsso_hip forward_train is a private tape-producing entry point and cannot "
            "participate in autograd directly; use lsso_amd.ball.hip.fast_mix()"
        )
    output, tape = _mixer_forward(
        projected, core_base_raw, core_drive_weight, eta_raw, centered_positions, valid_counts, True
    )
    assert tape is not None
    return output, tape


def backward(
    grad_output: torch.Tensor,
    projected: torch.Tensor,
    core_base_raw: torch.Tensor,
    core_drive_weight: torch.Tensor,
    eta_raw: torch.Tensor,
    tape: torch.Tensor,
    centered_positions: torch.Tensor | None = None,
    valid_counts: torch.Tensor | None = None,
    column_sums: bool = False,
):
    """Native first-order VJP of the mixer (csrc/ball/binding.cpp:92-95):
    returns (grad_projected, grad_core_base_raw, grad_core_drive_weight,
    grad_eta_raw), and with ``column_sums`` also the FP32 column sums of
    grad_projected over all rows (the input projection's bias gradient,
    taken inside the token map)."""

    library = _library()
    shape, mode = _validate_mixer(
        projected, core_base_raw, core_drive_weight, eta_raw, centered_positions, valid_counts
    )
    device = projected.device
    expected = (shape.batch, shape.length, shape.heads * shape.head_dim)
    if tuple(grad_output.shape) != expected:
        raise RuntimeError(f"grad_output must have shape {expected}, got {tuple(grad_output.shape)}")
    if grad_output.dtype != torch.bfloat16:
        raise RuntimeError("grad_output must use bfloat16 under the mixed precision HIP contract")
    _require_device_tensor(grad_output, "grad_output", device)
    _require_device_tensor(tape, "tape", device)
    grad_output = grad_output.contiguous()
    floats = ctypes.c_size_t()
    _check(library.lsso_hip_mixer_tape_floats(ctypes.byref(shape), ctypes.byref(floats)), library)
    if tape.dtype != torch.float32 or tape.numel() != floats.value or not tape.is_contiguous():
        raise RuntimeError("tape does not match this geometry's lsso_hip_mixer_tape_floats()")
    workspace_bytes = ctypes.c_size_t()
    _check(
        library.lsso_hip_mixer_backward_workspace_bytes(ctypes.byref(shape), mode, ctypes.byref(workspace_bytes)),
        library,
    )
    workspace = torch.empty(workspace_bytes.value, dtype=torch.uint8, device=device)
    grad_projected = torch.empty_like(projected)
    grad_base = torch.empty_like(core_base_raw)
    grad_drive = torch.empty_like(core_drive_weight)
    grad_eta = torch.empty_like(eta_raw)
    sums = torch.empty(projected.shape[-1], dtype=torch.float32, device=device) if column_sums else None
    with torch.cuda.device(device):
        status = library.lsso_hip_mixer_backward_ex(
            ctypes.byref(shape),
            grad_output.data_ptr(),
            projected.data_ptr(),
            core_base_raw.data_ptr(),
            core_drive_weight.data_ptr(),
            eta_raw.data_ptr(),
            ctypes.cast(_inverse_frequency(shape.rank), ctypes.c_void_p),
            None if centered_positions is None else centered_positions.data_ptr(),
            mode,
            None if valid_counts is None else valid_counts.data_ptr(),
            tape.data_ptr(),
            grad_projected.data_ptr(),
            grad_base.data_ptr(),
            grad_drive.data_ptr(),
            grad_eta.data_ptr(),
            None if sums is None else sums.data_ptr(),
            workspace.data_ptr(),
            workspace_bytes.value,
            _stream(device),
        )
    _check(status, library)
    if column_sums:
        return grad_projected, grad_base, grad_drive, grad_eta, sums
    return grad_projected, grad_base, grad_drive, grad_eta


class _FastMix(torch.autograd.Function):
    """First-order autograd boundary of the native mixer (cuda.py:220-280),
    calling the registered operators as the reference does."""

    @staticmethod
    def forward(ctx, projected, core_base_raw, core_drive_weight, eta_raw, centered_positions, valid_counts):
        output, tape, pivots = torch.ops.lsso_equilibrium.forward_train(
            projected, core_base_raw, core_drive_weight, eta_raw, centered_positions, valid_counts
        )
        ctx.save_for_backward(projected, core_base_raw, core_drive_weight, eta_raw, tape, pivots)
        ctx.centered_positions = centered_positions
        ctx.valid_counts = valid_counts
        return output

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, grad_output):
        projected, core_base_raw, core_drive_weight, eta_raw, tape, pivots = ctx.saved_tensors
        grads = torch.ops.lsso_equilibrium.backward(
            grad_output.to(dtype=torch.bfloat16).contiguous(),
            projected,
            core_base_raw,
            core_drive_weight,
            eta_raw,
            tape,
            pivots,
            ctx.centered_positions,
            ctx.valid_counts,
        )
        needs = ctx.needs_input_grad
        return (
            grads[0] if needs[0] else None,
            grads[1] if needs[1] else None,
            grads[2] if needs[2] else None,
            grads[3] if needs[3] else None,
            None,
            None,
        )


def fast_mix(
    projected: torch.Tensor,
    core_base_raw: torch.Tensor,
    core_drive_weight: torch.Tensor,
    eta_raw: torch.Tensor,
    centered_positions: torch.Tensor | None = None,
    valid_counts: torch.Tensor | None = None,
) -> torch.Tensor:
    """Run the strict native mixer, selecting the inference or training entry
    from autograd state (cuda.py:283-323)."""

    if centered_positions is not None and centered_positions.requires_grad:
        raise ValueError(
            "the LSSO HIP fast path does not support gradients for centered_positions"
        )
    if valid_counts is not None and valid_counts.requires_grad:
        raise ValueError("the LSSO HIP fast path does not support gradients for valid_counts")
    require_available()
    if not torch.is_grad_enabled() or not _any_requires_grad(
        projected, core_base_raw, core_drive_weight, eta_raw
    ):
        return torch.ops.lsso_equilibrium.forward_inference(
            projected, core_base_raw, core_drive_weight, eta_raw, centered_positions, valid_counts
        )
    return _FastMix.apply(
        projected, core_base_raw, core_drive_weight, eta_raw, centered_positions, valid_counts
    )


def mix_project_supported(
    projected: torch.Tensor,
    core_base_raw: torch.Tensor,
    core_drive_weight: torch.Tensor,
    eta_raw: torch.Tensor,
) -> bool:
    """Whether the fused mixer + output projection covers this geometry."""

    library = _library()
    shape, _mode = _validate_mixer(projected, core_base_raw, core_drive_weight, eta_raw, None, None)
    status = library.lsso_hip_mixer_projected_supported(ctypes.byref(shape))
    if status < 0:
        _check(status, library)
    return status == 1


def mix_project(
    projected: torch.Tensor,
    core_base_raw: torch.Tensor,
    core_drive_weight: torch.Tensor,
    eta_raw: torch.Tensor,
    centered_positions: torch.Tensor | None,
    valid_counts: torch.Tensor | None,
    out_weight: torch.Tensor,
    out_bias: torch.Tensor | None,
    output_dtype: torch.dtype,
    row_mask: torch.Tensor | None = None,
) -> torch.Tensor:
    """Inference-only native mixer fused with the biased output projection.

    Bitwise ``linear(forward_inference(...), out_weight, out_bias,
    output_dtype, row_mask)``: the mixed tensor stays on chip (the
    orchestration of reference model.py:389-405 in one pass).
    """

    if torch.is_grad_enabled() and _any_requires_grad(
        projected, core_base_raw, core_drive_weight, eta_raw, centered_positions, valid_counts,
        out_weight, out_bias,
    ):
        raise RuntimeError(
            "lsso_hip mix_project is an inference-only entry point and cannot participate in "
            "autograd; use fast_mix() followed by linear()"
        )
    library = _library()
    shape, mode = _validate_mixer(
        projected, core_base_raw, core_drive_weight, eta_raw, centered_positions, valid_counts
    )
    device = projected.device
    dim = shape.heads * shape.head_dim
    dtype_codes = {torch.float16: _F16, torch.bfloat16: _BF16}
    if output_dtype not in dtype_codes:
        raise TypeError("the fused projection supports float16/bfloat16 outputs")
    if out_weight.dtype != torch.float32 or tuple(out_weight.shape) != (dim, dim):
        raise TypeError(f"out_weight must be float32 [{dim}, {dim}]")
    if out_bias is not None and (out_bias.dtype != torch.float32 or tuple(out_bias.shape) != (dim,)):
        raise TypeError(f"out_bias must be float32 [{dim}]")
    for name, value in (("out_weight", out_weight), ("out_bias", out_bias)):
        if value is not None:
            _require_device_tensor(value, name, device)
    out_weight = out_weight.contiguous()
    out_bias = None if out_bias is None else out_bias.contiguous()
    mask_ptr = None
    if row_mask is not None:
        if row_mask.dtype != torch.bool or tuple(row_mask.shape) != (shape.batch, shape.length):
            raise ValueError("row_mask must be a bool [B, N] tensor")
        row_mask = row_mask.contiguous()
        mask_ptr = row_mask.data_ptr()
    workspace_bytes = ctypes.c_size_t()
    _check(library.lsso_hip_mixer_workspace_bytes(ctypes.byref(shape), mode, ctypes.byref(workspace_bytes)), library)
    workspace = torch.empty(workspace_bytes.value, dtype=torch.uint8, device=device)
    output = torch.empty((shape.batch, shape.length, dim), dtype=output_dtype, device=device)
    with torch.cuda.device(device):
        status = library.lsso_hip_mixer_forward_projected(
            ctypes.byref(shape),
            projected.data_ptr(),
            core_base_raw.data_ptr(),
            core_drive_weight.data_ptr(),
            eta_raw.data_ptr(),
            ctypes.cast(_inverse_frequency(shape.rank), ctypes.c_void_p),
            None if centered_positions is None else centered_positions.data_ptr(),
            mode,
            None if valid_counts is None else valid_counts.data_ptr(),
            out_weight.data_ptr(),
            None if out_bias is None else out_bias.data_ptr(),
            mask_ptr,
            output.data_ptr(),
            dtype_codes[output_dtype],
            workspace.data_ptr(),
            workspace_bytes.value,
            _stream(device),
        )
    _check(status, library)
    return output


def _layer_shape(
    x: torch.Tensor,
    in_weight: torch.Tensor,
    core_base_raw: torch.Tensor,
    core_drive_weight: torch.Tensor,
    eta_raw: torch.Tensor,
    centered_positions: torch.Tensor | None,
    valid_counts: torch.Tensor | None,
) -> tuple[MixerShape, int]:
    if x.device.type != "cuda":
        raise RuntimeError("x must be a CUDA (ROCm device) tensor")
    if x.dim() != 3 or not x.is_contiguous():
        raise RuntimeError(f"x must be a contiguous [B, N, D] tensor, got {tuple(x.shape)}")
    batch, length, dim = x.shape
    if core_base_raw.dim() != 3:
        raise RuntimeError(f"core_base_raw must have shape [H, R, R], got {tuple(core_base_raw.shape)}")
    width = core_base_raw.shape[0] * core_base_raw.shape[1] + dim
    if in_weight.dtype != torch.float32 or tuple(in_weight.shape) != (width, dim):
        raise TypeError(f"in_weight must be float32 [{width}, {dim}]")
    return _validate_core(
        x.device, batch, length, width, core_base_raw, core_drive_weight, eta_raw,
        centered_positions, valid_counts,
    )


def layer_supported(
    x: torch.Tensor,
    in_weight: torch.Tensor,
    core_base_raw: torch.Tensor,
    core_drive_weight: torch.Tensor,
    eta_raw: torch.Tensor,
) -> bool:
    """Whether the fused whole-layer forward covers this geometry."""

    library = _library()
    shape, _mode = _layer_shape(x, in_weight, core_base_raw, core_drive_weight, eta_raw, None, None)
    status = library.lsso_hip_layer_supported(ctypes.byref(shape))
    if status < 0:
        _check(status, library)
    return status == 1 and x.dtype in (torch.float16, torch.bfloat16)


def layer_forward(
    x: torch.Tensor,
    in_weight: torch.Tensor,
    in_bias: torch.Tensor | None,
    core_base_raw: torch.Tensor,
    core_drive_weight: torch.Tensor,
    eta_raw: torch.Tensor,
    centered_positions: torch.Tensor | None,
    valid_counts: torch.Tensor | None,
    out_weight: torch.Tensor,
    out_bias: torch.Tensor | None,
    row_mask: torch.Tensor | None = None,
    stage_events: list | None = None,
) -> torch.Tensor:
    """Inference-only native LSSO layer, x -> y, in one call.

    Bitwise ``linear(mix(linear(x, in_weight, in_bias, bf16, row_mask)),
    out_weight, out_bias, x.dtype, row_mask)``: the input projection runs fused
    with the token reductions and the output projection with the apply (the
    orchestration of reference model.py:270-405).

    ``stage_events``: optional 8 recorded ``torch.cuda.Event`` objects (or
    None); events 2k and 2k + 1 are recorded around stage k (phase table,
    projection + reductions, compact solve, apply + output projection), for
    per-kernel timing on the launch stream.
    """

    if torch.is_grad_enabled() and _any_requires_grad(
        x, in_weight, in_bias, core_base_raw, core_drive_weight, eta_raw, centered_positions,
        valid_counts, out_weight, out_bias,
    ):
        raise RuntimeError(
            "lsso_hip layer_forward is an inference-only entry point and cannot participate in "
            "autograd; use linear(), fast_mix() and linear()"
        )
    library = _library()
    shape, mode = _layer_shape(
        x, in_weight, core_base_raw, core_drive_weight, eta_raw, centered_positions, valid_counts
    )
    device = x.device
    dim = x.shape[-1]
    width = in_weight.shape[0]
    dtype_codes = {torch.float16: _F16, torch.bfloat16: _BF16}
    if x.dtype not in dtype_codes:
        raise TypeError("the fused layer supports float16/bfloat16 x")
    if in_bias is not None and (in_bias.dtype != torch.float32 or tuple(in_bias.shape) != (width,)):
        raise TypeError(f"in_bias must be float32 [{width}]")
    if out_weight.dtype != torch.float32 or tuple(out_weight.shape) != (dim, dim):
        raise TypeError(f"out_weight must be float32 [{dim}, {dim}]")
    if out_bias is not None and (out_bias.dtype != torch.float32 or tuple(out_bias.shape) != (dim,)):
        raise TypeError(f"out_bias must be float32 [{dim}]")
    for name, value in (
        ("in_weight", in_weight), ("in_bias", in_bias), ("out_weight", out_weight), ("out_bias", out_bias),
    ):
        if value is not None:
            _require_device_tensor(value, name, device)
    in_weight = in_weight.contiguous()
    in_bias = None if in_bias is None else in_bias.contiguous()
    out_weight = out_weight.contiguous()
    out_bias = None if out_bias is None else out_bias.contiguous()
    mask_ptr = None
    if row_mask is not None:
        if row_mask.dtype != torch.bool or tuple(row_mask.shape) != (shape.batch, shape.length):
            raise ValueError("row_mask must be a bool [B, N] tensor")
        row_mask = row_mask.contiguous()
        mask_ptr = row_mask.data_ptr()
    workspace_bytes = ctypes.c_size_t()
    _check(library.lsso_hip_layer_workspace_bytes(ctypes.byref(shape), mode, ctypes.byref(workspace_bytes)), library)
    workspace = torch.empty(workspace_bytes.value, dtype=torch.uint8, device=device)
    output = torch.empty((shape.batch, shape.length, dim), dtype=x.dtype, device=device)
    arguments = []
    entry = library.lsso_hip_layer_forward
    if stage_events is not None:
        if len(stage_events) != 8:
            raise ValueError("stage_events must hold 8 events (or None entries)")
        handles = []
        for event in stage_events:
            handle = 0 if event is None else int(event.cuda_event)
            if event is not None and handle == 0:
                raise ValueError("stage events must have been recorded once (torch creates them lazily)")
            handles.append(handle)
        arguments = [(ctypes.c_void_p * 8)(*[h or None for h in handles])]
        entry = library.lsso_hip_layer_forward_timed
    with torch.cuda.device(device):
        status = entry(
            ctypes.byref(shape),
            x.data_ptr(),
            dtype_codes[x.dtype],
            in_weight.data_ptr(),
            None if in_bias is None else in_bias.data_ptr(),
            mask_ptr,
            core_base_raw.data_ptr(),
            core_drive_weight.data_ptr(),
            eta_raw.data_ptr(),
            ctypes.cast(_inverse_frequency(shape.rank), ctypes.c_void_p),
            None if centered_positions is None else centered_positions.data_ptr(),
            mode,
            None if valid_counts is None else valid_counts.data_ptr(),
            out_weight.data_ptr(),
            None if out_bias is None else out_bias.data_ptr(),
            output.data_ptr(),
            dtype_codes[x.dtype],
            workspace.data_ptr(),
            workspace_bytes.value,
            _stream(device),
            *arguments,
        )
    _check(status, library)
    return output


def _project_mix_forward(
    x: torch.Tensor,
    in_weight: torch.Tensor,
    in_bias: torch.Tensor | None,
    core_base_raw: torch.Tensor,
    core_drive_weight: torch.Tensor,
    eta_raw: torch.Tensor,
    centered_positions: torch.Tensor | None,
    valid_counts: torch.Tensor | None,
    row_mask: torch.Tensor | None,
    record_tape: bool,
    out_weight: torch.Tensor | None = None,
    out_bias: torch.Tensor | None = None,
):
    """(packed, mixed, tape) of lsso_hip_project_mix_forward, or (packed,
    mixed, tape, y) of lsso_hip_layer_forward_train when ``out_weight`` is
    given (no autograd)."""

    library = _library()
    shape, mode = _layer_shape(
        x, in_weight, core_base_raw, core_drive_weight, eta_raw, centered_positions, valid_counts
    )
    device = x.device
    width = in_weight.shape[0]
    dtype_codes = {torch.float16: _F16, torch.bfloat16: _BF16}
    if x.dtype not in dtype_codes:
        raise TypeError("the fused projection + mixer supports float16/bfloat16 x")
    if in_bias is not None and (in_bias.dtype != torch.float32 or tuple(in_bias.shape) != (width,)):
        raise TypeError(f"in_bias must be float32 [{width}]")
    _require_device_tensor(in_weight, "in_weight", device)
    if in_bias is not None:
        _require_device_tensor(in_bias, "in_bias", device)
    in_weight = in_weight.contiguous()
    in_bias = None if in_bias is None else in_bias.contiguous()
    mask_ptr = None
    if row_mask is not None:
        if row_mask.dtype != torch.bool or tuple(row_mask.shape) != (shape.batch, shape.length):
            raise ValueError("row_mask must be a bool [B, N] tensor")
        row_mask = row_mask.contiguous()
        mask_ptr = row_mask.data_ptr()
    workspace_bytes = ctypes.c_size_t()
    _check(library.lsso_hip_mixer_workspace_bytes(ctypes.byref(shape), mode, ctypes.byref(workspace_bytes)), library)
    workspace = torch.empty(workspace_bytes.value, dtype=torch.uint8, device=device)
    packed = torch.empty((shape.batch, shape.length, width), dtype=torch.bfloat16, device=device)
    mixed = torch.empty(
        (shape.batch, shape.length, shape.heads * shape.head_dim), dtype=torch.bfloat16, device=device
    )
    tape = None
    if record_tape:
        floats = ctypes.c_size_t()
        _check(library.lsso_hip_mixer_tape_floats(ctypes.byref(shape), ctypes.byref(floats)), library)
        tape = torch.empty(floats.value, dtype=torch.float32, device=device)
    common = (
        ctypes.byref(shape),
        x.data_ptr(),
        dtype_codes[x.dtype],
        in_weight.data_ptr(),
        None if in_bias is None else in_bias.data_ptr(),
        mask_ptr,
        core_base_raw.data_ptr(),
        core_drive_weight.data_ptr(),
        eta_raw.data_ptr(),
        ctypes.cast(_inverse_frequency(shape.rank), ctypes.c_void_p),
        None if centered_positions is None else centered_positions.data_ptr(),
        mode,
        None if valid_counts is None else valid_counts.data_ptr(),
    )
    if out_weight is None:
        with torch.cuda.device(device):
            status = library.lsso_hip_project_mix_forward(
                *common,
                packed.data_ptr(),
                mixed.data_ptr(),
                None if tape is None else tape.data_ptr(),
                workspace.data_ptr(),
                workspace_bytes.value,
                _stream(device),
            )
        _check(status, library)
        return packed, mixed, tape
    dim = shape.heads * shape.head_dim
    if out_weight.dtype != torch.float32 or tuple(out_weight.shape) != (dim, dim):
        raise TypeError(f"out_weight must be float32 [{dim}, {dim}]")
    if out_bias is not None and (out_bias.dtype != torch.float32 or tuple(out_bias.shape) != (dim,)):
        raise TypeError(f"out_bias must be float32 [{dim}]")
    _require_device_tensor(out_weight, "out_weight", device)
    if out_bias is not None:
        _require_device_tensor(out_bias, "out_bias", device)
    out_weight = out_weight.contiguous()
    out_bias = None if out_bias is None else out_bias.contiguous()
    y = torch.empty((shape.batch, shape.length, dim), dtype=x.dtype, device=device)
    with torch.cuda.device(device):
        status = library.lsso_hip_layer_forward_train(
            *common,
            out_weight.data_ptr(),
            None if out_bias is None else out_bias.data_ptr(),
            packed.data_ptr(),
            mixed.data_ptr(),
            None if tape is None else tape.data_ptr(),
            y.data_ptr(),
            dtype_codes[x.dtype],
            workspace.data_ptr(),
            workspace_bytes.value,
            _stream(device),
        )
    _check(status, library)
    return packed, mixed, tape, y


class _ProjectMix(torch.autograd.Function):
    """Autograd of the input projection and the mixer run as one native call
    (lsso_hip_project_mix_forward).  The backward is the mixer VJP
    (cuda.py:256-280) followed by the projection VJP (reference.py:205-247),
    exactly as when the two run separately."""

    @staticmethod
    def forward(ctx, x, in_weight, in_bias, core_base_raw, core_drive_weight, eta_raw,
                centered_positions, valid_counts, row_mask):
        with torch.no_grad():
            packed, mixed, tape = _project_mix_forward(
                x, in_weight, in_bias, core_base_raw, core_drive_weight, eta_raw,
                centered_positions, valid_counts, row_mask, True,
            )
        ctx.save_for_backward(x, in_weight, packed, core_base_raw, core_drive_weight, eta_raw, tape, row_mask)
        ctx.centered_positions = centered_positions
        ctx.valid_counts = valid_counts
        ctx.has_bias = in_bias is not None
        ctx.bias_dtype = None if in_bias is None else in_bias.dtype
        return mixed

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, grad_mixed):
        x, in_weight, packed, core_base_raw, core_drive_weight, eta_raw, tape, row_mask = ctx.saved_tensors
        needs = ctx.needs_input_grad
        # Without a row mask, the column sums of grad_packed taken inside the
        # token map are the bias gradient.  With one, rows the mask excludes
        # must not count, and only the projection VJP's own pass knows them.
        need_bias = ctx.has_bias and needs[2]
        fused_sums = need_bias and row_mask is None
        grads = backward(
            grad_mixed.to(dtype=torch.bfloat16),
            packed,
            core_base_raw,
            core_drive_weight,
            eta_raw,
            tape,
            ctx.centered_positions,
            ctx.valid_counts,
            column_sums=fused_sums,
        )
        grad_packed, grad_base, grad_drive, grad_eta = grads[:4]
        grad_x, grad_weight, grad_bias = _linear_vjp(
            grad_packed, x, in_weight, row_mask, needs[0], needs[1], need_bias, ctx.bias_dtype,
            grads[4] if fused_sums else None,
        )
        return (
            grad_x,
            grad_weight,
            grad_bias,
            grad_base if needs[3] else None,
            grad_drive if needs[4] else None,
            grad_eta if needs[5] else None,
            None,
            None,
            None,
        )


def project_mix(
    x: torch.Tensor,
    in_weight: torch.Tensor,
    in_bias: torch.Tensor | None,
    core_base_raw: torch.Tensor,
    core_drive_weight: torch.Tensor,
    eta_raw: torch.Tensor,
    centered_positions: torch.Tensor | None = None,
    valid_counts: torch.Tensor | None = None,
    row_mask: torch.Tensor | None = None,
) -> torch.Tensor:
    """mixed = fast_mix(linear(x, in_weight, in_bias, bf16, row_mask), ...)
    in one native call, bitwise that of the two (the input projection runs
    fused with the token reductions).  Differentiable (first order) when
    autograd needs it; ask ``layer_supported`` first."""

    for name, value in (("centered_positions", centered_positions), ("valid_counts", valid_counts)):
        if value is not None and value.requires_grad:
            raise ValueError(f"the LSSO HIP fast path does not support gradients for {name}")
    require_available()
    if torch.is_grad_enabled() and _any_requires_grad(
        x, in_weight, in_bias, core_base_raw, core_drive_weight, eta_raw
    ):
        return _ProjectMix.apply(
            x, in_weight, in_bias, core_base_raw, core_drive_weight, eta_raw,
            centered_positions, valid_counts, row_mask,
        )
    _packed, mixed, _tape = _project_mix_forward(
        x, in_weight, in_bias, core_base_raw, core_drive_weight, eta_raw,
        centered_positions, valid_counts, row_mask, False,
    )
    return mixed


class _Layer(torch.autograd.Function):
    """Autograd of the whole layer run as one native training call
    (lsso_hip_layer_forward_train: input projection, mixer with the tape and
    output projection).  The backward is the output projection's VJP
    (reference.py:205-247), the mixer VJP (cuda.py:256-280) and the input
    projection's VJP, exactly as when the three run separately."""

    @staticmethod
    def forward(ctx, x, in_weight, in_bias, core_base_raw, core_drive_weight, eta_raw,
                out_weight, out_bias, centered_positions, valid_counts, row_mask):
        with torch.no_grad():
            packed, mixed, tape, y = _project_mix_forward(
                x, in_weight, in_bias, core_base_raw, core_drive_weight, eta_raw,
                centered_positions, valid_counts, row_mask, True, out_weight, out_bias,
            )
        ctx.save_for_backward(x, in_weight, packed, core_base_raw, core_drive_weight, eta_raw, tape,
                              row_mask, mixed, out_weight)
        ctx.centered_positions = centered_positions
        ctx.valid_counts = valid_counts
        ctx.in_bias_dtype = None if in_bias is None else in_bias.dtype
        ctx.out_bias_dtype = None if out_bias is None else out_bias.dtype
        return y

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, grad_y):
        (x, in_weight, packed, core_base_raw, core_drive_weight, eta_raw, tape, row_mask, mixed,
         out_weight) = ctx.saved_tensors
        needs = ctx.needs_input_grad
        need_mixer = any(needs[:6])
        grad_mixed, grad_out_weight, grad_out_bias = _linear_vjp(
            grad_y, mixed, out_weight, row_mask, need_mixer, needs[6],
            ctx.out_bias_dtype is not None and needs[7], ctx.out_bias_dtype,
        )
        grad_x = grad_in_weight = grad_in_bias = grad_base = grad_drive = grad_eta = None
        if need_mixer:
            need_in_bias = ctx.in_bias_dtype is not None and needs[2]
            fused_sums = need_in_bias and row_mask is None
            grads = backward(
                grad_mixed.to(dtype=torch.bfloat16),
                packed,
                core_base_raw,
                core_drive_weight,
                eta_raw,
                tape,
                ctx.centered_positions,
                ctx.valid_counts,
                column_sums=fused_sums,
            )
            grad_packed, grad_base, grad_drive, grad_eta = grads[:4]
            grad_x, grad_in_weight, grad_in_bias = _linear_vjp(
                grad_packed, x, in_weight, row_mask, needs[0], needs[1], need_in_bias,
                ctx.in_bias_dtype, grads[4] if fused_sums else None,
            )
        return (
            grad_x,
            grad_in_weight,
            grad_in_bias,
            grad_base if needs[3] else None,
            grad_drive if needs[4] else None,
            grad_eta if needs[5] else None,
            grad_out_weight,
            grad_out_bias,
            None,
            None,
            None,
        )


def layer_train(
    x: torch.Tensor,
    in_weight: torch.Tensor,
    in_bias: torch.Tensor | None,
    core_base_raw: torch.Tensor,
    core_drive_weight: torch.Tensor,
    eta_raw: torch.Tensor,
    out_weight: torch.Tensor,
    out_bias: torch.Tensor | None,
    centered_positions: torch.Tensor | None = None,
    valid_counts: torch.Tensor | None = None,
    row_mask: torch.Tensor | None = None,
) -> torch.Tensor:
    """y = linear(project_mix(x, ...), out_weight, out_bias, x.dtype, row_mask)
    in one native call (lsso_hip_layer_forward_train), bitwise that of the
    two, with the apply and the output projection in one kernel inside the
    fused readout's envelope.  Differentiable (first order); ask
    ``layer_supported`` first."""

    for name, value in (("centered_positions", centered_positions), ("valid_counts", valid_counts)):
        if value is not None and value.requires_grad:
            raise ValueError(f"the LSSO HIP fast path does not support gradients for {name}")
    require_available()
    if torch.is_grad_enabled() and _any_requires_grad(
        x, in_weight, in_bias, core_base_raw, core_drive_weight, eta_raw, out_weight, out_bias
    ):
        return _Layer.apply(
            x, in_weight, in_bias, core_base_raw, core_drive_weight, eta_raw, out_weight, out_bias,
            centered_positions, valid_counts, row_mask,
        )
    return _project_mix_forward(
        x, in_weight, in_bias, core_base_raw, core_drive_weight, eta_raw,
        centered_positions, valid_counts, row_mask, False, out_weight, out_bias,
    )[3]


def _rows(value: torch.Tensor, features: int) -> torch.Tensor:
    """value as a [rows, features] matrix whose rows the native kernels can
    address: unit feature stride and a row stride of at least `features`.
    Broadcast views (an expanded input, or the upstream gradient of a sum,
    whose row stride is 0) and other overlapping layouts are copied."""

    flat = value.reshape(-1, features)
    if flat.shape[0] > 1 and (flat.stride(-1) != 1 or flat.stride(0) < features):
        flat = flat.contiguous()
    elif flat.shape[0] <= 1 and flat.stride(-1) != 1:
        flat = flat.contiguous()
    return flat


def _linear_forward(
    value: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor | None,
    output_dtype: torch.dtype,
    row_mask: torch.Tensor | None = None,
) -> torch.Tensor:
    """The native projection kernel (no autograd)."""

    library = _library()
    if value.device.type != "cuda":
        raise RuntimeError("value must be a CUDA (ROCm device) tensor")
    dtype_codes = {torch.float16: _F16, torch.bfloat16: _BF16}
    if value.dtype not in dtype_codes or output_dtype not in dtype_codes:
        raise TypeError("the HIP projection supports float16/bfloat16 activations and outputs")
    if weight.dtype != torch.float32 or weight.dim() != 2:
        raise TypeError("the HIP projection requires a float32 [out, in] weight")
    if bias is not None and (bias.dtype != torch.float32 or tuple(bias.shape) != (weight.shape[0],)):
        raise TypeError("the HIP projection requires a float32 [out] bias")
    weight = weight.contiguous()
    bias = None if bias is None else bias.contiguous()
    in_features = value.shape[-1]
    if weight.shape[1] != in_features:
        raise ValueError(
            f"projection input and weight features must agree, got {in_features} and {weight.shape[1]}"
        )
    flat = _rows(value, in_features)
    rows = flat.shape[0]
    out_features = weight.shape[0]
    output = torch.empty(value.shape[:-1] + (out_features,), dtype=output_dtype, device=value.device)
    mask_ptr = None
    if row_mask is not None:
        if row_mask.dtype != torch.bool or tuple(row_mask.shape) != tuple(value.shape[:-1]):
            raise ValueError("row_mask must be a bool tensor shaped like the leading dimensions")
        row_mask = row_mask.contiguous()
        mask_ptr = row_mask.data_ptr()
    with torch.cuda.device(value.device):
        status = library.lsso_hip_linear(
            flat.data_ptr(),
            dtype_codes[value.dtype],
            rows,
            in_features,
            flat.stride(0) if rows > 1 else in_features,
            weight.data_ptr(),
            None if bias is None else bias.data_ptr(),
            mask_ptr,
            out_features,
            output.data_ptr(),
            dtype_codes[output_dtype],
            None,
            0,
            _stream(value.device),
        )
    _check(status, library)
    return output




def _grad_columns(
    flat: torch.Tensor,
    row_mask: torch.Tensor | None,
    want_copy: bool,
    want_sums: bool,
) -> tuple[torch.Tensor | None, torch.Tensor | None]:
    """One native pass over a [rows, cols] float16/bfloat16 gradient (or
    activation): its BF16 copy with ``row_mask``-excluded rows zeroed, and its
    FP32 column sums over the kept rows (the bias gradient)."""

    library = _library()
    rows, cols = flat.shape
    dtype_codes = {torch.float16: _F16, torch.bfloat16: _BF16}
    copy = torch.empty((rows, cols), dtype=torch.bfloat16, device=flat.device) if want_copy else None
    sums = torch.empty(cols, dtype=torch.float32, device=flat.device) if want_sums else None
    workspace = None
    size = ctypes.c_size_t(0)
    if want_sums:
        _check(library.lsso_hip_linear_grad_columns_workspace_bytes(rows, cols, ctypes.byref(size)), library)
        workspace = torch.empty(max(size.value, 1), dtype=torch.uint8, device=flat.device)
    mask = None if row_mask is None else row_mask.reshape(-1).contiguous()
    with torch.cuda.device(flat.device):
        status = library.lsso_hip_linear_grad_columns(
            flat.data_ptr(),
            dtype_codes[flat.dtype],
            rows,
            cols,
            flat.stride(0) if rows > 1 else cols,
            None if mask is None else mask.data_ptr(),
            None if copy is None else copy.data_ptr(),
            None if sums is None else sums.data_ptr(),
            None if workspace is None else workspace.data_ptr(),
            size.value,
            _stream(flat.device),
        )
    _check(status, library)
    return copy, sums


def _weight_gradient(
    flat_grad: torch.Tensor,
    flat_value: torch.Tensor,
    row_mask: torch.Tensor | None,
    want_bias: bool,
) -> tuple[torch.Tensor, torch.Tensor | None]:
    """FP32 [out, in] = sum over rows of bf16(grad)^T bf16(value), and (when
    asked) the FP32 column sums of grad, on the native weight-gradient kernel
    (one pass over both operands, rows excluded by ``row_mask`` count as
    zero, deterministic)."""

    library = _library()
    rows, out_features = flat_grad.shape
    in_features = flat_value.shape[1]
    dtype_codes = {torch.float16: _F16, torch.bfloat16: _BF16}
    device = flat_grad.device
    grad_weight = torch.empty((out_features, in_features), dtype=torch.float32, device=device)
    grad_bias = torch.empty(out_features, dtype=torch.float32, device=device) if want_bias else None
    size = ctypes.c_size_t(0)
    _check(library.lsso_hip_linear_weight_grad_workspace_bytes(
        rows, in_features, out_features, ctypes.byref(size)), library)
    workspace = torch.empty(max(size.value, 1), dtype=torch.uint8, device=device)
    mask = None if row_mask is None else row_mask.reshape(-1).contiguous()
    with torch.cuda.device(device):
        status = library.lsso_hip_linear_weight_grad(
            flat_grad.data_ptr(),
            dtype_codes[flat_grad.dtype],
            flat_grad.stride(0) if rows > 1 else out_features,
            flat_value.data_ptr(),
            dtype_codes[flat_value.dtype],
            flat_value.stride(0) if rows > 1 else in_features,
            rows,
            in_features,
            out_features,
            None if mask is None else mask.data_ptr(),
            grad_weight.data_ptr(),
            None if grad_bias is None else grad_bias.data_ptr(),
            workspace.data_ptr(),
            size.value,
            _stream(device),
        )
    _check(status, library)
    return grad_weight, grad_bias


class _Linear(torch.autograd.Function):
    """Autograd of the native projection with the reference's VJP
    (lsso/ball/reference.py:205-247): BF16 operands with FP32 accumulation
    for the value and weight gradients, an FP32 sum of the upstream gradient
    for the bias.  The value gradient runs on the native projection kernel
    (dX = bf16(dY) bf16(W), stored once in the value's dtype), the weight and
    bias gradients on the native weight-gradient kernel, which reads dY and
    the value in their own dtypes.  Rows excluded by ``row_mask`` carry no
    gradient."""

    @staticmethod
    def forward(ctx, value, weight, bias, output_dtype, row_mask):
        output = _linear_forward(value, weight, bias, output_dtype, row_mask)
        ctx.save_for_backward(value, weight, row_mask)
        ctx.has_bias = bias is not None
        ctx.bias_dtype = None if bias is None else bias.dtype
        return output

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, grad_output):
        value, weight, row_mask = ctx.saved_tensors
        grad_value, grad_weight, grad_bias = _linear_vjp(
            grad_output, value, weight, row_mask, ctx.needs_input_grad[0],
            ctx.needs_input_grad[1], ctx.has_bias and ctx.needs_input_grad[2], ctx.bias_dtype,
        )
        return grad_value, grad_weight, grad_bias, None, None


def _linear_vjp(
    grad_output: torch.Tensor,
    value: torch.Tensor,
    weight: torch.Tensor,
    row_mask: torch.Tensor | None,
    need_value: bool,
    need_weight: bool,
    need_bias: bool,
    bias_dtype: torch.dtype | None,
    grad_sums: torch.Tensor | None = None,
):
    """(dX, dW, db) of y = cast(bf16(x) bf16(W)^T + b) (reference.py:205-247).
    ``grad_sums``: the FP32 column sums of dY when the caller already has
    them (over the rows ``row_mask`` keeps), so no pass over dY is made for
    the bias.

    dX runs on the native projection kernel from dY in its own dtype with the
    transposed weight; dW (and db when it is still needed) on the native
    weight-gradient kernel, which reads dY and x in their own dtypes; a bias
    gradient alone takes one native column-sum pass over dY."""

    out_features, in_features = weight.shape
    flat_grad = _rows(grad_output, out_features)
    if flat_grad.dtype not in (torch.float16, torch.bfloat16):
        flat_grad = flat_grad.to(dtype=torch.bfloat16).contiguous()
    grad_value = grad_weight = grad_bias = None
    if need_value:
        grad_value = _linear_forward(
            flat_grad, weight.mT.contiguous(), None, value.dtype,
            None if row_mask is None else row_mask.reshape(-1),
        ).reshape(value.shape)
    sums_needed = need_bias and grad_sums is None
    if need_weight:
        flat_value = _rows(value, in_features)
        if flat_value.dtype not in (torch.float16, torch.bfloat16):
            raise TypeError("the HIP projection supports float16/bfloat16 activations")
        grad_weight, computed = _weight_gradient(flat_grad, flat_value, row_mask, sums_needed)
        grad_weight = grad_weight.to(dtype=weight.dtype)
        if sums_needed:
            grad_sums = computed
    elif sums_needed:
        _, grad_sums = _grad_columns(flat_grad, row_mask, False, True)
    if need_bias:
        grad_bias = grad_sums.to(dtype=bias_dtype)
    return grad_value, grad_weight, grad_bias


def linear(
    value: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor | None,
    output_dtype: torch.dtype,
    row_mask: torch.Tensor | None = None,
) -> torch.Tensor:
    """Native biased projection cast(bf16(x) bf16(W)^T + b) (reference.py:20-75, 347-408).

    value: [..., K] float16/bfloat16 with unit feature stride; weight: float32
    [N, K]; bias: float32 [N] or None; output: contiguous [..., N].
    ``row_mask`` (bool, value.shape[:-1]) zeroes the output rows it excludes.
    Differentiable (first order) when autograd needs it.
    """

    if torch.is_grad_enabled() and _any_requires_grad(value, weight, bias):
        return _Linear.apply(value, weight, bias, output_dtype, row_mask)
    return _linear_forward(value, weight, bias, output_dtype, row_mask)


__all__ = [
    "backward",
    "fast_mix",
    "forward_inference",
    "forward_train",
    "is_available",
    "layer_forward",
    "layer_train",
    "layer_supported",
    "linear",
    "load",
    "mix_project",
    "mix_project_supported",
    "project_mix",
    "require_available",
]
