"""Canonical LSSO mathematics in plain PyTorch (``implementation="reference"``).

This is the framework's device-agnostic path for every core mode and ablation;
the gfx950 library serves ``implementation="hip"``.  It follows the operator
contract of the reference (lsso/ball/reference.py, docs/CORE_CONTRACT.md) with
one deliberate engineering choice: the QR soft frame is evaluated through its
Gram-Cholesky identity.  For A in R^{N x r}, QR([A/s; I/s]) has
R_qr^T R_qr = (A^T A + I) / s^2, so with L L^T = A^T A + I (positive diagonal,
the reference's sign convention) R_qr = L^T / s and P = (A/s) R_qr^-1 =
A L^-T.  The detached scale s cancels; no (N + r) x r factorization is run.

Numerics of the FP32 path match the reference CPU branch: FP32 projections,
BF16 rounding of the packed coordinates and of the pre-output mix, FP16-stored
rotary phases, FP32 frame/solve.  FP64 inputs run entirely in FP64.
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as functional

_RANK_PHASE_BASE = 10000.0
_SOFTPLUS_ONE_OFFSET = math.log(math.expm1(1.0))


def _calculation_dtype(value: torch.Tensor) -> torch.dtype:
    return torch.float64 if value.dtype == torch.float64 else torch.float32


def linear(
    value: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor | None = None,
    *,
    output_dtype: torch.dtype | None = None,
) -> torch.Tensor:
    """FP32 (FP64 for FP64 operands) projection with bias, then one cast.

    Reference: tensor_core_linear CPU branch (lsso/ball/reference.py:404-408).
    """

    calc = torch.float64 if (value.dtype == torch.float64 or weight.dtype == torch.float64) else torch.float32
    output = torch.matmul(value.to(calc), weight.to(calc).mT)
    if bias is not None:
        output = output + bias.to(device=output.device, dtype=output.dtype)
    return output if output_dtype is None else output.to(output_dtype)


def rotary_inverse_frequency(rank: int, dtype: torch.dtype, device: torch.device | None = None) -> torch.Tensor:
    """Rank-Rotary frequencies 10000^(-j / (rank/2)) (reference.py:704-707)."""

    half = rank // 2
    return _RANK_PHASE_BASE ** (-torch.arange(half, device=device, dtype=dtype) / half)


def rank_rotary(relation: torch.Tensor, positions: torch.Tensor) -> torch.Tensor:
    """Rotate rank pairs (2j, 2j+1) by positions * 10000^(-j/(r/2)).

    relation: [B, H, N, R]; positions: [B, N].  Non-FP64 phases are computed
    in FP32 and stored as FP16 (reference.py:691-724).
    """

    if relation.ndim != 4:
        raise ValueError("relation must have shape [B, H, N, R]")
    batch, _heads, length, rank = relation.shape
    if positions.shape != (batch, length):
        raise ValueError(
            f"positions must have shape {(batch, length)}, got {tuple(positions.shape)}"
        )
    if rank % 2:
        raise ValueError(f"Rank-Rotary requires an even rank, got rank={rank}")
    half = rank // 2
    angles = positions[:, :, None] * rotary_inverse_frequency(rank, relation.dtype, relation.device)[None, None, :]
    cos = angles.cos()
    sin = angles.sin()
    if relation.dtype != torch.float64:
        cos = cos.to(torch.float16).to(relation.dtype)
        sin = sin.to(torch.float16).to(relation.dtype)
    cos = cos.view(batch, 1, length, half)
    sin = sin.view(batch, 1, length, half)
    even = relation[..., 0::2]
    odd = relation[..., 1::2]
    return torch.stack((even * cos - odd * sin, even * sin + odd * cos), dim=-1).flatten(-2)


def qr_soft_frame(relation: torch.Tensor) -> torch.Tensor:
    """Soft frame P = A L^-T with L L^T = A^T A + I (equal to the reference's
    positive-diagonal QR frame of [A/s; I/s], reference.py:411-447)."""

    if relation.ndim < 2:
        raise ValueError("relation must have at least two matrix dimensions")
    if not relation.is_floating_point():
        raise TypeError("relation must be a floating-point tensor")
    value = relation.to(_calculation_dtype(relation))
    length, rank = value.shape[-2:]
    if length == 0 or rank == 0:
        return value
    eye = torch.eye(rank, dtype=value.dtype, device=value.device)
    factor = torch.linalg.cholesky(value.mT @ value + eye)
    return torch.linalg.solve_triangular(factor, value.mT, upper=False).mT


def bounded_complement(raw: torch.Tensor) -> torch.Tensor:
    """eta = (1 - eps) tanh(raw) by sign-split logistic identities (reference.py:450-471)."""

    if not raw.is_floating_point():
        raise TypeError("complement coordinates must be a floating-point tensor")
    calc = _calculation_dtype(raw)
    value = raw.to(calc)
    scale = 1.0 - torch.finfo(calc).eps
    positive_exponent = torch.exp(-2.0 * torch.clamp_min(value, 0.0))
    negative_exponent = torch.exp(2.0 * torch.clamp_max(value, 0.0))
    positive = (1.0 - positive_exponent) / (1.0 + positive_exponent)
    negative = (negative_exponent - 1.0) / (1.0 + negative_exponent)
    return scale * torch.where(value >= 0.0, positive, negative)


def accretive_generator(raw: torch.Tensor) -> torch.Tensor:
    """K = F F^T + Omega: F = tril(raw, -1) + diag(softplus(diag raw + log(e-1))),
    Omega = triu(raw, 1) - triu(raw, 1)^T (reference.py:474-497)."""

    if raw.ndim < 2 or raw.shape[-2] != raw.shape[-1]:
        raise ValueError("raw must be square in its final two dimensions")
    value = raw.to(_calculation_dtype(raw))
    diagonal = torch.diagonal(value, dim1=-2, dim2=-1)
    factor = torch.tril(value, diagonal=-1) + torch.diag_embed(
        functional.softplus(diagonal + _SOFTPLUS_ONE_OFFSET)
    )
    upper = torch.triu(value, diagonal=1)
    return factor @ factor.mT + (upper - upper.mT)


def accretive_equilibrium_mix(
    frame: torch.Tensor,
    generator: torch.Tensor | None,
    compact_state: torch.Tensor,
    content: torch.Tensor,
    eta: torch.Tensor,
) -> torch.Tensor:
    """Y = eta C + P [2 (I + K)^-1 Z - (1 + eta) Z]; ZERO core: Y = eta (C - P Z)
    (reference.py:500-572)."""

    heads = frame.shape[1]
    eta_batch = eta.view(1, heads, 1, 1)
    if generator is None:
        compact = -eta_batch * compact_state
    else:
        rank = frame.shape[-1]
        if generator.ndim == 3:
            generator = generator.unsqueeze(0).expand(frame.shape[0], -1, -1, -1)
        identity = torch.eye(rank, dtype=content.dtype, device=content.device)
        equilibrium = torch.linalg.solve(generator + identity, compact_state)
        compact = 2.0 * equilibrium - (1.0 + eta_batch) * compact_state
    return eta_batch * content + frame @ compact


def _equilibrium_certificates(
    frame_gram: torch.Tensor,
    system: torch.Tensor,
    compact_state: torch.Tensor,
    eta: torch.Tensor,
    adjoint_rhs: torch.Tensor,
    length: int,
) -> dict[str, torch.Tensor]:
    """FP64 certificates of T = eta I_N + P (2 (I + K)^-1 - I - eta I_r) P^T
    given only compact quantities: P^T P, I + K, Z and the adjoint RHS."""

    rank = system.shape[-1]
    heads = system.shape[1]
    identity = torch.eye(rank, dtype=torch.float64, device=system.device)
    eta = eta.view(1, heads)
    # Restricted to range(P), T acts as eta I + S^1/2 V^T (Refl - eta I) V S^1/2
    # in the eigenbasis P^T P = V S V^T; on range(P)'s complement it is eta I.
    values, vectors = torch.linalg.eigh(frame_gram)
    root_values = values.clamp_min(0.0).sqrt()
    reflection = 2.0 * torch.linalg.solve(system, identity.expand_as(system)) - identity
    eta_identity = eta[..., None, None] * identity
    block = eta_identity + root_values[..., :, None] * (
        vectors.mT @ (reflection - eta_identity) @ vectors
    ) * root_values[..., None, :]
    gain = torch.linalg.svdvals(block)[..., 0]
    if length > rank:
        gain = torch.maximum(gain, eta.abs())
    mu = torch.linalg.eigvalsh(0.5 * (system + system.mT))[..., 0]
    tiny = torch.finfo(torch.float64).tiny
    state = torch.linalg.solve(system, compact_state)
    adjoint = torch.linalg.solve(system.mT, adjoint_rhs)
    state_ratio = torch.linalg.vector_norm(state, dim=(-2, -1)) / torch.linalg.vector_norm(
        compact_state, dim=(-2, -1)
    ).clamp_min(tiny)
    adjoint_ratio = torch.linalg.vector_norm(adjoint, dim=(-2, -1)) / torch.linalg.vector_norm(
        adjoint_rhs, dim=(-2, -1)
    ).clamp_min(tiny)
    return {
        "q": gain,
        "contraction_slack": 1.0 - gain,
        "mu": mu,
        "state_ratio": state_ratio,
        "adjoint_ratio": adjoint_ratio,
        "state_bound_usage": mu * state_ratio,
        "adjoint_bound_usage": mu * adjoint_ratio,
    }


def compact_equilibrium_diagnostics(
    frame: torch.Tensor,
    generator: torch.Tensor,
    compact_state: torch.Tensor,
    eta: torch.Tensor,
    adjoint_rhs: torch.Tensor,
) -> dict[str, torch.Tensor]:
    """Realized token gain q = ||T||_2, the accretivity floor mu =
    lambda_min(sym(I + K)) and the solve / adjoint ratios, all [B, H] and in
    FP64 (reference.py:575-688).  The N x N operator is never formed: its
    norm follows from the R x R certificate block (requires N >= R)."""

    if frame.ndim != 4:
        raise ValueError("frame must have shape [B, H, N, R]")
    if generator.ndim not in (3, 4):
        raise ValueError("generator must have shape [H, R, R] or [B, H, R, R]")
    if compact_state.ndim != 4 or adjoint_rhs.ndim != 4:
        raise ValueError("compact_state and adjoint_rhs must have shape [B, H, R, D]")
    batch, heads, length, rank = frame.shape
    if length < rank:
        raise ValueError(
            f"compact diagnostics require sequence length N >= rank R, got N={length}, R={rank}"
        )
    state_shape = (batch, heads, rank, compact_state.shape[-1])
    if tuple(compact_state.shape) != state_shape:
        raise ValueError(f"compact_state must have shape {state_shape}, got {tuple(compact_state.shape)}")
    if adjoint_rhs.shape != compact_state.shape:
        raise ValueError(
            f"adjoint_rhs must match compact_state, got {tuple(adjoint_rhs.shape)} and "
            f"{tuple(compact_state.shape)}"
        )
    if tuple(eta.shape) != (heads,):
        raise ValueError(f"eta must have shape [{heads}], got {tuple(eta.shape)}")
    if generator.ndim == 3:
        if tuple(generator.shape) != (heads, rank, rank):
            raise ValueError(
                f"static generator must have shape {(heads, rank, rank)}, got {tuple(generator.shape)}"
            )
        generator = generator.unsqueeze(0).expand(batch, -1, -1, -1)
    elif tuple(generator.shape) != (batch, heads, rank, rank):
        raise ValueError(
            f"dynamic generator must have shape {(batch, heads, rank, rank)}, got {tuple(generator.shape)}"
        )
    others = (generator, compact_state, eta, adjoint_rhs)
    if any(value.device != frame.device for value in others):
        raise ValueError("all diagnostic inputs must share a device")
    if any(not value.is_floating_point() for value in (frame, *others)):
        raise TypeError("all diagnostic inputs must be floating-point tensors")
    with torch.autocast(device_type=frame.device.type, enabled=False):
        frame64 = frame.to(dtype=torch.float64)
        identity = torch.eye(rank, dtype=torch.float64, device=frame.device)
        return _equilibrium_certificates(
            frame64.mT @ frame64,
            generator.to(dtype=torch.float64) + identity,
            compact_state.to(dtype=torch.float64),
            eta.to(dtype=torch.float64),
            adjoint_rhs.to(dtype=torch.float64),
            length,
        )


__all__ = [
    "accretive_equilibrium_mix",
    "accretive_generator",
    "bounded_complement",
    "compact_equilibrium_diagnostics",
    "linear",
    "qr_soft_frame",
    "rank_rotary",
    "rotary_inverse_frequency",
]
