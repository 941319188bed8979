"""``torch.library`` registration of the reference's native operator schemas.

The reference's CUDA extension registers the namespace ``lsso_equilibrium``
with four operators when its shared object is loaded
(csrc/ball/binding.cpp:79-107), and its Python boundary calls them through
``torch.ops.lsso_equilibrium`` (lsso/ball/cuda.py:231, 269, 305).  ``register()``
defines the same schemas, backed by the gfx950 library's C ABI through
``lsso_amd.ball.hip``, so that code written against ``torch.ops`` runs on
MI355X unchanged, and so that ``torch.compile`` traces the operators through
the fake implementations below instead of breaking the graph at a ctypes call.
``lsso_amd.ball.hip.load()`` calls it once the library is loaded, as the
reference registers its operators inside ``load()``.

Differences from the reference that callers can observe:
- ``contract_version()`` returns the HIP library's C-ABI contract version,
  not the CUDA extension's.
- The tape holds compact per-system state only (no token-sized frame); the
  library needs no LU pivots, so ``forward_train`` returns a zero-length
  int32 ``pivots`` tensor and ``backward`` accepts and ignores it.
"""

from __future__ import annotations

from threading import Lock

import torch

NAMESPACE = "lsso_equilibrium"

# The reference's schemas, verbatim (csrc/ball/binding.cpp:80-95).
SCHEMAS = {
    "contract_version": "contract_version() -> int",
    "forward_inference": (
        "forward_inference(Tensor projected, Tensor core_base_raw, Tensor core_drive_weight, "
        "Tensor eta_raw, Tensor? centered_positions=None, Tensor? valid_counts=None) -> Tensor"
    ),
    "forward_train": (
        "forward_train(Tensor projected, Tensor core_base_raw, Tensor core_drive_weight, "
        "Tensor eta_raw, Tensor? centered_positions=None, Tensor? valid_counts=None) "
        "-> (Tensor, Tensor, Tensor)"
    ),
    "backward": (
        "backward(Tensor grad_output, Tensor projected, Tensor core_base_raw, "
        "Tensor core_drive_weight, Tensor eta_raw, Tensor tape, Tensor pivots, "
        "Tensor? centered_positions=None, Tensor? valid_counts=None) "
        "-> (Tensor, Tensor, Tensor, Tensor)"
    ),
}

_REGISTER_LOCK = Lock()
_LIBRARY_DEF: torch.library.Library | None = None


def _any_requires_grad(*values: torch.Tensor | None) -> bool:
    return any(value is not None and value.requires_grad for value in values)


def _contract_version() -> int:
    from . import hip

    return int(hip._library().lsso_hip_contract_version())


def _forward_inference(projected, core_base_raw, core_drive_weight, eta_raw,
                       centered_positions=None, valid_counts=None):
    from . import hip

    output, _tape = hip._mixer_forward(
        projected, core_base_raw, core_drive_weight, eta_raw, centered_positions, valid_counts, False
    )
    return output


def _forward_train(projected, core_base_raw, core_drive_weight, eta_raw,
                   centered_positions=None, valid_counts=None):
    from . import hip

    output, tape = hip._mixer_forward(
        projected, core_base_raw, core_drive_weight, eta_raw, centered_positions, valid_counts, True
    )
    pivots = torch.empty((0,), dtype=torch.int32, device=projected.device)
    return output, tape, pivots


def _backward(grad_output, projected, core_base_raw, core_drive_weight, eta_raw, tape, pivots,
              centered_positions=None, valid_counts=None):
    from . import hip

    del pivots  # the Gauss-Jordan solve keeps no pivots on the tape
    return tuple(hip.backward(
        grad_output, projected, core_base_raw, core_drive_weight, eta_raw, tape,
        centered_positions, valid_counts,
    ))


def _guarded(name: str, message: str):
    """Autograd-key kernel that rejects a differentiable call, as the
    reference's forward_*_autograd do (binding.cpp:16-70), then redispatches
    below autograd."""

    def kernel(keyset, projected, core_base_raw, core_drive_weight, eta_raw,
               centered_positions=None, valid_counts=None):
        if torch.is_grad_enabled() and _any_requires_grad(
            projected, core_base_raw, core_drive_weight, eta_raw, centered_positions, valid_counts
        ):
            raise RuntimeError(message)
        operator = getattr(getattr(torch.ops, NAMESPACE), name).default
        return operator.redispatch(
            keyset & torch._C._after_autograd_keyset, projected, core_base_raw, core_drive_weight,
            eta_raw, centered_positions, valid_counts,
        )

    return kernel


def _geometry(projected: torch.Tensor, core_base_raw: torch.Tensor) -> tuple[int, int, int, int, int]:
    if projected.dim() != 3 or core_base_raw.dim() != 3:
        raise RuntimeError("projected must be [B, N, H*R + D] and core_base_raw [H, R, R]")
    batch, length, width = projected.shape
    heads, rank = core_base_raw.shape[0], core_base_raw.shape[1]
    if width <= heads * rank or (width - heads * rank) % heads:
        raise RuntimeError("projected width must be H*R plus a content width divisible by H")
    return batch, length, heads, rank, (width - heads * rank) // heads


def _fake_forward_inference(projected, core_base_raw, core_drive_weight, eta_raw,
                            centered_positions=None, valid_counts=None):
    batch, length, heads, _rank, head_dim = _geometry(projected, core_base_raw)
    return projected.new_empty((batch, length, heads * head_dim), dtype=torch.bfloat16)


def _fake_forward_train(projected, core_base_raw, core_drive_weight, eta_raw,
                        centered_positions=None, valid_counts=None):
    batch, length, heads, rank, head_dim = _geometry(projected, core_base_raw)
    output = projected.new_empty((batch, length, heads * head_dim), dtype=torch.bfloat16)
    # Per system: L, Theta, (I + K)^-1 and L^-1 (r x r each), then Z and U
    # (r x d each); the same count as lsso_hip_mixer_tape_floats.
    tape = projected.new_empty((batch * heads * (4 * rank * rank + 2 * rank * head_dim),),
                               dtype=torch.float32)
    pivots = projected.new_empty((0,), dtype=torch.int32)
    return output, tape, pivots


def _fake_backward(grad_output, projected, core_base_raw, core_drive_weight, eta_raw, tape, pivots,
                   centered_positions=None, valid_counts=None):
    return (
        torch.empty_like(projected),
        torch.empty_like(core_base_raw),
        torch.empty_like(core_drive_weight),
        torch.empty_like(eta_raw),
    )


def is_registered() -> bool:
    """Whether this process's ``torch.ops.lsso_equilibrium`` holds the
    operators registered here."""

    return _LIBRARY_DEF is not None


def register() -> None:
    """Define ``lsso_equilibrium::{contract_version, forward_inference,
    forward_train, backward}`` once per process, with device kernels for the
    CUDA (ROCm) dispatch key, autograd guards for the two forwards and fake
    implementations for tracing."""

    global _LIBRARY_DEF
    with _REGISTER_LOCK:
        if _LIBRARY_DEF is not None:
            return
        library = torch.library.Library(NAMESPACE, "DEF")
        for schema in SCHEMAS.values():
            library.define(schema)
        library.impl("contract_version", _contract_version, "CompositeExplicitAutograd")
        library.impl("forward_inference", _forward_inference, "CUDA")
        library.impl("forward_train", _forward_train, "CUDA")
        library.impl("backward", _backward, "CUDA")
        library.impl(
            "forward_inference",
            _guarded("forward_inference",
                     "lsso_equilibrium::forward_inference is an inference-only entry point and "
                     "cannot participate in autograd directly; use lsso_amd.ball.hip.fast_mix()"),
            "Autograd",
            with_keyset=True,
        )
        library.impl(
            "forward_train",
            _guarded("forward_train",
                     "lsso_equilibrium::forward_train is a private tape-producing entry point and "
                     "cannot participate in autograd directly; use lsso_amd.ball.hip.fast_mix()"),
            "Autograd",
            with_keyset=True,
        )
        torch.library.register_fake(f"{NAMESPACE}::forward_inference", _fake_forward_inference, lib=library)
        torch.library.register_fake(f"{NAMESPACE}::forward_train", _fake_forward_train, lib=library)
        torch.library.register_fake(f"{NAMESPACE}::backward", _fake_backward, lib=library)
        _LIBRARY_DEF = library


__all__ = ["NAMESPACE", "SCHEMAS", "is_registered", "register"]
