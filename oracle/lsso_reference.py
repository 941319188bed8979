"""CPU oracle for the LSSO mixer -- TEST INFRASTRUCTURE ONLY.

This module restates, operation for operation, the reference PyTorch CPU path
of Yang916-yy/LSSO (lsso/ball/reference.py, lsso/ball/model.py) and the
ABI-level FP64 oracle of its native tests (tests/cuda/test_fast_path.py:33-86).
Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg may import it, and only as the checker or the timed CPU baseline; the
``lsso_amd`` package never imports it.

Pinning (see tests/test_oracle.py):
  * golden fixtures written by the real reference in this container
    (tests/golden/make_golden.py) pin the FP32 and FP64 module outputs, the
    packed projection, frame, compact state, generator and the ABI oracle;
  * closed forms pin the math independently: the frame identity
    P P^T = A (I + A^T A)^-1 A^T, the default-init point K = I (Y = eta (C -
    P P^T C)), the dense N x N operator on tiny inputs, rotation norm
    preservation, and the numpy Gram-Cholesky restatement
    (oracle/gram_cholesky.py) agreeing to ~1e-12 in FP64.
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as functional

RANK_PHASE_BASE = 10000.0
SOFTPLUS_ONE_OFFSET = math.log(math.expm1(1.0))
ETA_INIT_RAW = math.atanh(0.9)


def calculation_dtype(value: torch.Tensor) -> torch.dtype:
    return torch.float64 if value.dtype == torch.float64 else torch.float32


def linear_cpu(value, weight, bias=None, *, output_dtype=None):
    """tensor_core_linear on CPU: FP32 (or FP64) matmul, + bias, one cast.
    Reference: lsso/ball/reference.py:323-328, 404-408."""

    if value.dtype == torch.float64 or weight.dtype == torch.float64:
        output = torch.matmul(value.to(torch.float64), weight.mT.to(torch.float64))
    else:
        output = torch.matmul(value.to(torch.float32), weight.mT.to(torch.float32))
    if bias is not None:
        output = output + bias.to(dtype=output.dtype)
    return output if output_dtype is None else output.to(dtype=output_dtype)


def rank_rotary(relation: torch.Tensor, positions: torch.Tensor) -> torch.Tensor:
    """Reference: lsso/ball/reference.py:691-724."""

    batch, _heads, length, rank = relation.shape
    half = rank // 2
    inv_freq = RANK_PHASE_BASE ** (
        -torch.arange(half, device=relation.device, dtype=relation.dtype) / half
    )
    angles = positions[:, :, None] * inv_freq[None, None, :]
    cos = angles.cos()
    sin = angles.sin()
    if relation.dtype != torch.float64:
        cos = cos.to(torch.float16).to(relation.dtype)
        sin = sin.to(torch.float16).to(relation.dtype)
    cos = cos.view(batch, 1, length, half)
    sin = sin.view(batch, 1, length, half)
    even = relation[..., 0::2]
    odd = relation[..., 1::2]
    output = torch.empty_like(relation)
    output[..., 0::2] = even * cos - odd * sin
    output[..., 1::2] = even * sin + odd * cos
    return output


def qr_soft_frame(relation: torch.Tensor) -> torch.Tensor:
    """Reference: lsso/ball/reference.py:411-447 (detached scale, identity
    augmentation, reduced QR, positive-diagonal sign fix)."""

    value = relation.to(dtype=calculation_dtype(relation))
    length, rank = value.shape[-2:]
    scale = value.abs().amax(dim=(-2, -1), keepdim=True).clamp_min(1.0)
    eye = torch.eye(rank, dtype=value.dtype, device=value.device)
    augmented = torch.cat(
        (value / scale, eye.expand(value.shape[:-2] + (rank, rank)) / scale), dim=-2
    )
    orthogonal, factor = torch.linalg.qr(augmented, mode="reduced")
    diagonal = torch.diagonal(factor, dim1=-2, dim2=-1)
    signs = torch.where(diagonal < 0, -torch.ones_like(diagonal), torch.ones_like(diagonal))
    return (orthogonal * signs.unsqueeze(-2))[..., :length, :]


def bounded_complement(raw: torch.Tensor) -> torch.Tensor:
    """Reference: lsso/ball/reference.py:450-471."""

    calc = calculation_dtype(raw)
    value = raw.to(dtype=calc)
    interior = 1.0 - torch.finfo(calc).eps
    pe = torch.exp(-2.0 * torch.clamp_min(value, 0.0))
    ne = torch.exp(2.0 * torch.clamp_max(value, 0.0))
    positive = (1.0 - pe) / (1.0 + pe)
    negative = (ne - 1.0) / (1.0 + ne)
    return interior * torch.where(value >= 0.0, positive, negative)


def accretive_generator(raw: torch.Tensor) -> torch.Tensor:
    """Reference: lsso/ball/reference.py:474-497 (CPU F F^T in the calc dtype)."""

    value = raw.to(dtype=calculation_dtype(raw))
    diagonal = torch.diagonal(value, dim1=-2, dim2=-1)
    factor = torch.tril(value, diagonal=-1) + torch.diag_embed(
        functional.softplus(diagonal + SOFTPLUS_ONE_OFFSET)
    )
    upper = torch.triu(value, diagonal=1)
    return torch.matmul(factor, factor.mT) + (upper - upper.mT)


def accretive_equilibrium_mix(frame, generator, compact_state, content, eta):
    """Reference: lsso/ball/reference.py:500-572 (CPU matmul branch)."""

    heads = frame.shape[1]
    rank = frame.shape[-1]
    eta_batch = eta.view(1, heads, 1, 1)
    if generator is None:
        compact = -eta_batch * compact_state
    else:
        if generator.ndim == 3:
            generator = generator.unsqueeze(0).expand(frame.shape[0], -1, -1, -1)
        identity = torch.eye(rank, dtype=content.dtype, device=content.device)
        equilibrium = torch.linalg.solve(generator + identity, compact_state)
        compact = 2.0 * equilibrium - (1.0 + eta_batch) * compact_state
    return eta_batch * content + torch.matmul(frame, compact)


def center_positions(position_ids, valid_mask, *, dtype, all_valid, batch=None, length=None):
    """Reference: lsso/ball/model.py:163-243."""

    if valid_mask is not None:
        batch, length = valid_mask.shape
    if position_ids is None:
        positions = torch.arange(length, dtype=dtype).view(1, length).expand(batch, length)
    else:
        if position_ids.is_floating_point():
            position_dtype = torch.float64 if position_ids.dtype == torch.float64 else dtype
            positions = position_ids.to(dtype=position_dtype)
        else:
            positions = position_ids.to(dtype=torch.int64)
        if positions.ndim == 1:
            positions = positions.view(1, length).expand(batch, length)
    if all_valid:
        centered = positions - positions[:, :1]
        if centered.dtype == torch.int64:
            centered = centered.to(dtype=dtype)
        centered = centered - centered.mean(dim=-1, keepdim=True)
        return centered.to(dtype=dtype)
    first_valid = valid_mask.to(dtype=torch.int64).argmax(dim=-1, keepdim=True)
    anchor = positions.gather(dim=1, index=first_valid)
    centered = positions - anchor
    if centered.dtype == torch.int64:
        centered = centered.to(dtype=dtype)
    weights = valid_mask.to(dtype=centered.dtype)
    count = weights.sum(dim=-1, keepdim=True).clamp_min(1.0)
    safe = torch.where(valid_mask, centered, torch.zeros_like(centered))
    mean = (safe * weights).sum(dim=-1, keepdim=True) / count
    return torch.where(valid_mask, centered - mean, torch.zeros_like(centered)).to(dtype=dtype)


def fast_mix_fp64(projected, core_base_raw, core_drive_weight, eta_raw,
                  centered_positions=None, valid_counts=None):
    """FP64 ABI oracle of the native mixer: packed [B, N, H*R + D] -> mixed
    [B, N, D].  Reference: tests/cuda/test_fast_path.py:33-86 (default
    positions arange(N) - (N - 1) / 2)."""

    calc = torch.float64
    projected = projected.to(dtype=calc)
    core_base_raw = core_base_raw.to(dtype=calc)
    core_drive_weight = core_drive_weight.to(dtype=calc)
    eta_raw = eta_raw.to(dtype=calc)
    batch, length, width = projected.shape
    heads = core_base_raw.shape[0]
    rank = core_base_raw.shape[-1]
    dim = width - heads * rank
    head_dim = dim // heads
    if valid_counts is None:
        counts = torch.full((batch,), float(length), dtype=calc)
    else:
        counts = valid_counts.to(dtype=calc)
    if centered_positions is None:
        positions = torch.arange(length, dtype=calc) - 0.5 * (length - 1)
    else:
        positions = centered_positions.to(dtype=calc)
    relation, content = projected.split((heads * rank, dim), dim=-1)
    relation = relation.view(batch, length, heads, rank).transpose(1, 2)
    content = content.view(batch, length, heads, head_dim).transpose(1, 2)
    relation = rank_rotary(relation, positions.expand(batch, -1)) / counts.sqrt().view(batch, 1, 1, 1)
    frame = qr_soft_frame(relation)
    compact_state = frame.mT @ content
    coordinates = core_base_raw.unsqueeze(0) + (
        compact_state @ core_drive_weight / counts.sqrt().view(batch, 1, 1, 1)
    )
    return accretive_equilibrium_mix(
        frame, accretive_generator(coordinates), compact_state, content, bounded_complement(eta_raw)
    ).transpose(1, 2).contiguous().view(batch, length, dim)


def compact_problem(params, config, x, valid_mask=None, position_ids=None):
    """Reference: lsso/ball/model.py:407-496 on CPU.  ``params`` maps the
    reference state_dict names to tensors; ``config`` holds dim, num_heads,
    rank, core_mode ("dynamic"/"static"/"zero") and rank_rotary."""

    dim = config["dim"]
    heads = config["num_heads"]
    rank = config["rank"]
    head_dim = dim // heads
    batch, length, _ = x.shape
    all_valid = valid_mask is None
    safe_x = x if all_valid else torch.where(valid_mask[:, :, None], x, torch.zeros_like(x))
    projected = linear_cpu(
        safe_x,
        params["w_bc.weight"],
        params.get("w_bc.bias"),
        output_dtype=torch.float64 if x.dtype == torch.float64 else torch.bfloat16,
    )
    relation, content = projected.split((heads * rank, dim), dim=-1)
    relation = relation.view(batch, length, heads, rank).transpose(1, 2)
    content = content.view(batch, length, heads, head_dim).transpose(1, 2)
    if not all_valid:
        active = valid_mask[:, None, :, None]
        relation = torch.where(active, relation, torch.zeros_like(relation))
        content = torch.where(active, content, torch.zeros_like(content))
    calc = torch.float64 if x.dtype == torch.float64 else torch.float32
    relation = relation.to(dtype=calc)
    content = content.to(dtype=calc)
    if config.get("rank_rotary", True):
        centered = center_positions(
            position_ids, valid_mask, dtype=calc, all_valid=all_valid, batch=batch, length=length
        )
        relation = rank_rotary(relation, centered)
    valid_count = (
        torch.full((batch,), float(length), dtype=calc)
        if all_valid
        else valid_mask.sum(dim=-1).to(dtype=calc).clamp_min(1.0)
    )
    relation = relation / valid_count.sqrt().view(batch, 1, 1, 1)
    frame = qr_soft_frame(relation)
    compact_state = torch.matmul(frame.mT.to(calc), content.to(calc))
    mode = config.get("core_mode", "dynamic")
    if mode == "dynamic":
        dynamic = torch.matmul(compact_state, params["core_drive_weight"].to(dtype=calc))
        coordinates = params["core_base_raw"].to(dtype=calc).unsqueeze(0) + dynamic / valid_count.sqrt().view(-1, 1, 1, 1)
    elif mode == "static":
        coordinates = params["core_base_raw"].to(dtype=calc)
    else:
        coordinates = None
    generator = None if coordinates is None else accretive_generator(coordinates)
    eta = bounded_complement(params["eta_raw"]).to(dtype=calc)
    return projected, frame, compact_state, content, generator, eta


def lsso_forward(params, config, x, valid_mask=None, position_ids=None):
    """LSSO.forward(implementation="reference") on CPU (lsso/ball/model.py:542-585)."""

    batch, length, dim = x.shape
    projected, frame, compact_state, content, generator, eta = compact_problem(
        params, config, x, valid_mask, position_ids
    )
    output = accretive_equilibrium_mix(frame, generator, compact_state, content, eta)
    mixed = output
    if x.dtype != torch.float64:
        mixed = mixed.to(torch.bfloat16)
    mixed = mixed.transpose(1, 2).contiguous().view(batch, length, dim)
    output = linear_cpu(mixed, params["w_o.weight"], params.get("w_o.bias"), output_dtype=x.dtype)
    if valid_mask is not None:
        output = torch.where(valid_mask[:, :, None], output, torch.zeros_like(output))
    return output


def init_params(config, *, seed=None, generator=None):
    """State of a freshly constructed reference LSSO (lsso/ball/model.py:40-72):
    two nn.Linear layers drawn in construction order, zero compact core and
    eta_raw = atanh(0.9).  Consumes torch's global RNG like the reference when
    ``seed`` is given."""

    if seed is not None:
        torch.manual_seed(seed)
    dim = config["dim"]
    heads = config["num_heads"]
    rank = config["rank"]
    bias = config.get("bias", False)
    w_bc = torch.nn.Linear(dim, heads * rank + dim, bias=bias)
    w_o = torch.nn.Linear(dim, dim, bias=bias)
    params = {"w_bc.weight": w_bc.weight.detach().clone(), "w_o.weight": w_o.weight.detach().clone()}
    if bias:
        params["w_bc.bias"] = w_bc.bias.detach().clone()
        params["w_o.bias"] = w_o.bias.detach().clone()
    mode = config.get("core_mode", "dynamic")
    if mode in ("dynamic", "static"):
        params["core_base_raw"] = torch.zeros(heads, rank, rank)
    if mode == "dynamic":
        params["core_drive_weight"] = torch.zeros(heads, dim // heads, rank)
    params["eta_raw"] = torch.full((heads,), ETA_INIT_RAW, dtype=torch.float32)
    return params
