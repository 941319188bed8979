"""The LSSO module: parameters, checkpoint contract, masks/positions, dispatch.

Mirrors the reference module (lsso/ball/model.py:29-596): identical parameter
names, shapes, initialization order and ``_extra_state`` contract (version
12), so reference checkpoints load unchanged.  ``implementation`` selects the
device-agnostic PyTorch path ("reference", the default) or the gfx950 native
path ("hip"; "cuda" is accepted as the same request because ROCm PyTorch
names its devices "cuda").  The native path never falls back.
"""

from __future__ import annotations

import math

import torch
import torch.nn as nn

from .config import CoreMode, LSSOConfig
from . import reference as canonical

_CONTRACT_VERSION = 12
_ETA_INIT = 0.9
_ETA_INIT_RAW = math.atanh(_ETA_INIT)
_SUPPORTED_ACTIVATION_DTYPES = frozenset(
    (torch.float16, torch.bfloat16, torch.float32, torch.float64)
)
_NATIVE_IMPLEMENTATIONS = ("hip", "cuda")


class LSSO(nn.Module):
    """The accretive-equilibrium low-rank token mixer."""

    def __init__(self, config: LSSOConfig) -> None:
        super().__init__()
        self.config = config
        self.w_bc = nn.Linear(
            config.dim, config.num_heads * config.rank + config.dim, bias=config.bias
        )
        self.w_o = nn.Linear(config.dim, config.dim, bias=config.bias)
        if config.core_mode is CoreMode.DYNAMIC:
            self.core_base_raw = nn.Parameter(
                torch.zeros(config.num_heads, config.rank, config.rank)
            )
            self.core_drive_weight = nn.Parameter(
                torch.zeros(config.num_heads, config.head_dim, config.rank)
            )
        elif config.core_mode is CoreMode.STATIC:
            self.core_base_raw = nn.Parameter(
                torch.zeros(config.num_heads, config.rank, config.rank)
            )
            self.register_parameter("core_drive_weight", None)
        else:
            self.register_parameter("core_base_raw", None)
            self.register_parameter("core_drive_weight", None)
        self.eta_raw = nn.Parameter(
            torch.full((config.num_heads,), _ETA_INIT_RAW, dtype=torch.float32)
        )

    # -- checkpoint contract (reference model.py:74-140) --------------------
    def complement(self) -> torch.Tensor:
        """The learned per-head complement eta."""

        return canonical.bounded_complement(self.eta_raw)

    def _contract_state(self) -> dict[str, object]:
        config = self.config
        return {
            "version": _CONTRACT_VERSION,
            "operator": "accretive_equilibrium",
            "dim": config.dim,
            "num_heads": config.num_heads,
            "rank": config.rank,
            "core_mode": config.core_mode.value,
            "rank_rotary": config.rank_rotary,
            "eta_parameterization": "per_head_interior_tanh",
            "numerics": "tf32-wbc-ieee-fgram-tc16-v6",
            "bias": config.bias,
        }

    def get_extra_state(self) -> dict[str, object]:
        return self._contract_state()

    def set_extra_state(self, state: object) -> None:
        expected = self._contract_state()
        if not isinstance(state, dict):
            raise RuntimeError("LSSO checkpoint is missing its configuration contract")
        if state != expected:
            keys = sorted(set(state) | set(expected))
            mismatches = ", ".join(
                f"{key}: checkpoint={state.get(key)!r}, model={expected.get(key)!r}"
                for key in keys
                if state.get(key) != expected.get(key)
            )
            raise RuntimeError(f"incompatible LSSO checkpoint contract ({mismatches})")

    def _load_from_state_dict(
        self,
        state_dict,
        prefix,
        local_metadata,
        strict,
        missing_keys,
        unexpected_keys,
        error_msgs,
    ) -> None:
        contract_key = f"{prefix}_extra_state"
        if contract_key not in state_dict:
            error_msgs.append(
                f"LSSO checkpoint is missing its configuration contract ({contract_key!r})"
            )
        super()._load_from_state_dict(
            state_dict, prefix, local_metadata, strict, missing_keys, unexpected_keys, error_msgs
        )

    # -- masks and positions (reference model.py:142-243) -------------------
    @staticmethod
    def _validate_mask(
        valid_mask: torch.Tensor | None, *, batch: int, length: int, device: torch.device
    ) -> torch.Tensor:
        if valid_mask is None:
            return torch.ones(batch, length, dtype=torch.bool, device=device)
        if valid_mask.shape != (batch, length):
            raise ValueError(
                f"valid_mask must have shape {(batch, length)}, got {tuple(valid_mask.shape)}"
            )
        if valid_mask.dtype != torch.bool:
            raise TypeError(f"valid_mask must have dtype torch.bool, got {valid_mask.dtype}")
        return valid_mask.to(device=device)

    @staticmethod
    def _center_positions(
        position_ids: torch.Tensor | None,
        valid_mask: torch.Tensor | None,
        *,
        dtype: torch.dtype,
        all_valid: bool,
        batch: int | None = None,
        length: int | None = None,
        device: torch.device | None = None,
    ) -> torch.Tensor:
        """Positions relative to the first valid token, minus the valid mean.

        Integer ids are differenced before the float cast; float64 ids are
        centered in float64; float16/bfloat16 ids are rejected.
        """

        if valid_mask is None:
            if not all_valid:
                raise ValueError("valid_mask is required when tokens are masked")
            if batch is None or length is None or device is None:
                raise ValueError("batch, length, and device are required without valid_mask")
        else:
            batch, length = valid_mask.shape
            device = valid_mask.device
        if position_ids is None:
            positions = torch.arange(length, device=device, dtype=dtype)
            positions = positions.view(1, length).expand(batch, length)
        else:
            if position_ids.is_floating_point():
                if position_ids.dtype not in (torch.float32, torch.float64):
                    raise TypeError(
                        "floating position_ids must use torch.float32 or torch.float64, "
                        f"got {position_ids.dtype}"
                    )
                position_dtype = torch.float64 if position_ids.dtype == torch.float64 else dtype
                positions = position_ids.to(device=device, dtype=position_dtype)
            else:
                if position_ids.dtype == torch.bool or position_ids.is_complex():
                    raise TypeError(
                        "position_ids must use an integer dtype, torch.float32, or "
                        f"torch.float64, got {position_ids.dtype}"
                    )
                positions = position_ids.to(device=device, dtype=torch.int64)
            if positions.ndim == 1:
                if positions.numel() != length:
                    raise ValueError(
                        f"position_ids length {positions.numel()} must match N={length}"
                    )
                positions = positions.view(1, length).expand(batch, length)
            elif positions.shape != (batch, length):
                raise ValueError(
                    "position_ids must be None, [N], or "
                    f"[B, N]={batch, length}; got {tuple(positions.shape)}"
                )
        if all_valid:
            centered = positions - positions[:, :1]
            if centered.dtype == torch.int64:
                centered = centered.to(dtype=dtype)
            centered = centered - centered.mean(dim=-1, keepdim=True)
            return centered.to(dtype=dtype)
        assert valid_mask is not None
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

    # -- compact coordinates (reference model.py:245-268) -------------------
    def _compact_coordinates(
        self, compact_state: torch.Tensor, valid_count: torch.Tensor
    ) -> torch.Tensor | None:
        config = self.config
        if config.core_mode is CoreMode.DYNAMIC:
            if self.core_base_raw is None or self.core_drive_weight is None:
                raise RuntimeError("dynamic compact parameters are missing")
            dynamic = compact_state @ self.core_drive_weight.to(dtype=compact_state.dtype)
            base = self.core_base_raw.to(dtype=compact_state.dtype).unsqueeze(0)
            return base + dynamic / valid_count.sqrt().view(-1, 1, 1, 1)
        if config.core_mode is CoreMode.STATIC:
            if self.core_base_raw is None:
                raise RuntimeError("static compact parameters are missing")
            return self.core_base_raw.to(dtype=compact_state.dtype)
        return None

    # -- native gfx950 path (reference model.py:270-405) --------------------
    def _forward_native(
        self,
        x: torch.Tensor,
        valid_mask: torch.Tensor | None,
        position_ids: torch.Tensor | None,
        implementation: str,
    ) -> torch.Tensor:
        config = self.config
        if (
            config.core_mode is not CoreMode.DYNAMIC
            or not config.rank_rotary
            or config.rank not in (16, 32, 48, 64)
        ):
            raise ValueError(
                f"implementation={implementation!r} requires core_mode='dynamic', "
                "rank_rotary=True, and rank in {16, 32, 48, 64}"
            )
        if position_ids is not None and position_ids.requires_grad:
            raise ValueError(
                f"implementation={implementation!r} does not support gradients for position_ids"
            )
        if x.device.type != "cuda":
            raise ValueError(
                f"implementation={implementation!r} requires x to be a CUDA tensor "
                "(a ROCm device tensor)"
            )
        if x.dtype not in (torch.float16, torch.bfloat16):
            raise TypeError(
                f"implementation={implementation!r} supports x with dtype torch.float16 or "
                f"torch.bfloat16; got {x.dtype}"
            )
        if self.core_base_raw is None or self.core_drive_weight is None:
            raise RuntimeError("dynamic compact parameters are missing")
        for name, parameter in self.named_parameters():
            if parameter.device != x.device:
                raise RuntimeError(
                    f"implementation={implementation!r} requires {name} on {x.device}, "
                    f"got {parameter.device}"
                )
        for name, parameter in (
            ("w_bc.weight", self.w_bc.weight),
            ("w_bc.bias", self.w_bc.bias),
            ("w_o.weight", self.w_o.weight),
            ("w_o.bias", self.w_o.bias),
            ("core_base_raw", self.core_base_raw),
            ("core_drive_weight", self.core_drive_weight),
            ("eta_raw", self.eta_raw),
        ):
            if parameter is None:
                continue
            if parameter.dtype != torch.float32:
                raise TypeError(
                    f"implementation={implementation!r} requires {name} to use "
                    f"torch.float32, got {parameter.dtype}"
                )
            if not parameter.is_contiguous():
                raise RuntimeError(f"implementation={implementation!r} requires contiguous {name}")

        from . import hip

        needs_grad = torch.is_grad_enabled() and any(
            parameter.requires_grad for parameter in (x, *self.parameters())
        )
        if not needs_grad and x.is_contiguous() and hip.layer_supported(
            x, self.w_bc.weight, self.core_base_raw, self.core_drive_weight, self.eta_raw
        ):
            # Inference: the whole layer in one native call (input projection
            # fused with the reductions, apply with the output projection),
            # bitwise equal to the three-step path below.
            centered_positions, valid_counts, mask = self._native_geometry(
                x, valid_mask, position_ids
            )
            return hip.layer_forward(
                x,
                self.w_bc.weight,
                self.w_bc.bias,
                self.core_base_raw,
                self.core_drive_weight,
                self.eta_raw,
                centered_positions,
                valid_counts,
                self.w_o.weight,
                self.w_o.bias,
                row_mask=mask,
            )
        if needs_grad and x.is_contiguous() and hip.layer_supported(
            x, self.w_bc.weight, self.core_base_raw, self.core_drive_weight, self.eta_raw
        ):
            # Training: the whole layer in one native call that also keeps
            # packed, mixed and the tape for the backward (the input
            # projection runs fused with the token reductions, the apply with
            # the output projection where the shapes allow), bitwise equal to
            # the separate linear + fast_mix + linear below.
            centered_positions, valid_counts, mask = self._native_geometry(
                x, valid_mask, position_ids
            )
            return hip.layer_train(
                x,
                self.w_bc.weight,
                self.w_bc.bias,
                self.core_base_raw,
                self.core_drive_weight,
                self.eta_raw,
                self.w_o.weight,
                self.w_o.bias,
                centered_positions,
                valid_counts,
                row_mask=mask,
            )
        projected, centered_positions, valid_counts, mask = self._native_inputs(
            x, valid_mask, position_ids
        )
        if not needs_grad and hip.mix_project_supported(
            projected, self.core_base_raw, self.core_drive_weight, self.eta_raw
        ):
            # Inference: the mixer and the output projection in one pass,
            # bitwise equal to the two-step path below.
            return hip.mix_project(
                projected,
                self.core_base_raw,
                self.core_drive_weight,
                self.eta_raw,
                centered_positions,
                valid_counts,
                self.w_o.weight,
                self.w_o.bias,
                x.dtype,
                row_mask=mask,
            )
        mixed = hip.fast_mix(
            projected,
            self.core_base_raw,
            self.core_drive_weight,
            self.eta_raw,
            centered_positions,
            valid_counts,
        )
        return hip.linear(mixed, self.w_o.weight, self.w_o.bias, x.dtype, row_mask=mask)

    # -- reference path (reference model.py:407-496, 562-585) ---------------
    def _native_inputs(
        self,
        x: torch.Tensor,
        valid_mask: torch.Tensor | None,
        position_ids: torch.Tensor | None,
    ):
        """Packed projection (native K1) and the mixer's positions / counts."""

        from . import hip

        centered_positions, valid_counts, mask = self._native_geometry(x, valid_mask, position_ids)
        # Masked rows are neither read nor biased: the projection writes zeros
        # there (reference model.py:371-383, 402-404).
        projected = hip.linear(x, self.w_bc.weight, self.w_bc.bias, torch.bfloat16, row_mask=mask)
        return projected, centered_positions, valid_counts, mask

    def _native_geometry(
        self,
        x: torch.Tensor,
        valid_mask: torch.Tensor | None,
        position_ids: torch.Tensor | None,
    ):
        """The mixer's centred positions, valid counts and row mask
        (reference model.py:270-370)."""

        batch, length, _dim = x.shape
        all_valid = valid_mask is None
        mask = (
            None
            if all_valid
            else self._validate_mask(valid_mask, batch=batch, length=length, device=x.device)
        )
        centered_positions = None
        if valid_mask is not None or position_ids is not None:
            centered = self._center_positions(
                position_ids,
                mask,
                dtype=torch.float32,
                all_valid=all_valid,
                batch=batch,
                length=length,
                device=x.device,
            )
            if position_ids is None or position_ids.ndim == 1:
                centered_positions = centered[0].contiguous() if all_valid else centered.contiguous()
            else:
                centered_positions = centered.contiguous()
        valid_counts = (
            None
            if all_valid
            else mask.sum(dim=-1).to(dtype=torch.float32).clamp_min(1.0).contiguous()
        )
        return centered_positions, valid_counts, mask

    @torch.no_grad()
    def diagnostics(
        self,
        x: torch.Tensor,
        valid_mask: torch.Tensor | None = None,
        position_ids: torch.Tensor | None = None,
        *,
        adjoint_rhs: torch.Tensor,
        implementation: str = "reference",
    ) -> dict[str, torch.Tensor]:
        """Per-sample, per-head FP64 certificates of the realized operator
        (reference model.py:498-522): token gain q, mu, solve/adjoint ratios.

        ``implementation="reference"`` realizes the compact problem with the
        canonical torch path, as the reference does.  ``"hip"`` (or
        ``"cuda"``) certifies the operator that the native kernels realize,
        from their compact tape: P^T P = I - L^-1 L^-T, I + K from Theta, Z.
        """

        self._validate_input(x)
        if self.config.core_mode is CoreMode.ZERO:
            raise ValueError("compact diagnostics require a nonzero compact core")
        if implementation == "reference":
            _projected, frame, compact_state, _content, generator, eta, _mask = (
                self._reference_compact_problem(x, valid_mask, position_ids)
            )
            assert generator is not None
            return canonical.compact_equilibrium_diagnostics(
                frame, generator, compact_state, eta,
                adjoint_rhs.to(device=x.device, dtype=compact_state.dtype),
            )
        if implementation not in ("hip", "cuda"):
            raise ValueError(
                "implementation must be 'reference', 'hip' or 'cuda', got " f"{implementation!r}"
            )
        if self.config.core_mode is not CoreMode.DYNAMIC or not self.config.rank_rotary:
            raise ValueError(
                f"implementation={implementation!r} diagnostics require the dynamic rank-rotary core"
            )
        from . import hip

        config = self.config
        batch, length, _dim = x.shape
        rank, heads, head_dim = config.rank, config.num_heads, config.head_dim
        if length < rank:
            raise ValueError(
                f"compact diagnostics require sequence length N >= rank R, got N={length}, R={rank}"
            )
        projected, positions, counts, _mask = self._native_inputs(x, valid_mask, position_ids)
        _mixed, tape = hip.forward_train(
            projected, self.core_base_raw, self.core_drive_weight, self.eta_raw, positions, counts
        )
        rr, rd = rank * rank, rank * head_dim
        tape = tape.view(batch, heads, 4 * rr + 2 * rd).double()
        linv = tape[..., 3 * rr:4 * rr].reshape(batch, heads, rank, rank)
        theta = tape[..., rr:2 * rr].reshape(batch, heads, rank, rank)
        compact_state = tape[..., 4 * rr:4 * rr + rd].reshape(batch, heads, rank, head_dim)
        identity = torch.eye(rank, dtype=torch.float64, device=x.device)
        frame_gram = identity - linv @ linv.mT
        system = identity + canonical.accretive_generator(theta)
        rhs = adjoint_rhs.to(device=x.device, dtype=torch.float64)
        if tuple(rhs.shape) != tuple(compact_state.shape):
            raise ValueError(
                f"adjoint_rhs must have shape {tuple(compact_state.shape)}, got {tuple(rhs.shape)}"
            )
        eta = self.complement().to(device=x.device, dtype=torch.float64)
        return canonical._equilibrium_certificates(frame_gram, system, compact_state, eta, rhs, length)

    def _reference_compact_problem(
        self,
        x: torch.Tensor,
        valid_mask: torch.Tensor | None,
        position_ids: torch.Tensor | None,
    ):
        config = self.config
        batch, length, _dim = x.shape
        all_valid = valid_mask is None
        mask = (
            None
            if all_valid
            else self._validate_mask(valid_mask, batch=batch, length=length, device=x.device)
        )
        safe_x = x if all_valid else torch.where(mask[:, :, None], x, torch.zeros_like(x))
        projected = canonical.linear(
            safe_x,
            self.w_bc.weight,
            self.w_bc.bias,
            output_dtype=torch.float64 if x.dtype == torch.float64 else torch.bfloat16,
        )
        relation, content = projected.split((config.num_heads * config.rank, config.dim), dim=-1)
        relation = relation.view(batch, length, config.num_heads, config.rank).transpose(1, 2)
        content = content.view(batch, length, config.num_heads, config.head_dim).transpose(1, 2)
        if not all_valid:
            active = mask[:, None, :, None]
            relation = torch.where(active, relation, torch.zeros_like(relation))
            content = torch.where(active, content, torch.zeros_like(content))
        calc_dtype = torch.float64 if x.dtype == torch.float64 else torch.float32
        with torch.autocast(device_type=x.device.type, enabled=False):
            relation = relation.to(dtype=calc_dtype)
            content = content.to(dtype=calc_dtype)
            if config.rank_rotary:
                centered = self._center_positions(
                    position_ids,
                    mask,
                    dtype=calc_dtype,
                    all_valid=all_valid,
                    batch=batch,
                    length=length,
                    device=x.device,
                )
                relation = canonical.rank_rotary(relation, centered)
            valid_count = (
                torch.full((batch,), float(length), dtype=calc_dtype, device=x.device)
                if all_valid
                else mask.sum(dim=-1).to(dtype=calc_dtype).clamp_min(1.0)
            )
            relation = relation / valid_count.sqrt().view(batch, 1, 1, 1)
            frame = canonical.qr_soft_frame(relation)
            compact_state = frame.mT @ content
            coordinates = self._compact_coordinates(compact_state, valid_count)
            generator = None if coordinates is None else canonical.accretive_generator(coordinates)
            eta = self.complement().to(device=x.device, dtype=calc_dtype)
        return projected, frame, compact_state, content, generator, eta, mask

    def _validate_input(self, x: torch.Tensor) -> None:
        config = self.config
        if x.ndim != 3 or x.shape[-1] != config.dim:
            raise ValueError(f"x must have shape [B, N, {config.dim}], got {tuple(x.shape)}")
        if not x.is_floating_point():
            raise TypeError("x must be a floating-point tensor")
        if x.dtype not in _SUPPORTED_ACTIVATION_DTYPES:
            raise TypeError(
                f"LSSO does not support x with dtype {x.dtype}; use torch.float16, "
                "torch.bfloat16, torch.float32, or torch.float64"
            )
        if x.shape[0] == 0:
            raise ValueError("batch size must be positive")
        if x.shape[1] == 0:
            raise ValueError("sequence length must be positive")

    def forward(
        self,
        x: torch.Tensor,
        valid_mask: torch.Tensor | None = None,
        position_ids: torch.Tensor | None = None,
        *,
        implementation: str = "reference",
    ) -> torch.Tensor:
        self._validate_input(x)
        config = self.config
        batch, length, _dim = x.shape
        if implementation in _NATIVE_IMPLEMENTATIONS:
            return self._forward_native(x, valid_mask, position_ids, implementation)
        if implementation != "reference":
            raise ValueError(
                "implementation must be 'reference', 'hip' or 'cuda', "
                f"got {implementation!r}"
            )
        _projected, frame, compact_state, content, generator, eta, mask = (
            self._reference_compact_problem(x, valid_mask, position_ids)
        )
        with torch.autocast(device_type=x.device.type, enabled=False):
            output = canonical.accretive_equilibrium_mix(frame, generator, compact_state, content, eta)
        if x.dtype != torch.float64:
            output = output.to(torch.bfloat16)
        output = output.transpose(1, 2).contiguous().view(batch, length, config.dim)
        output = canonical.linear(output, self.w_o.weight, self.w_o.bias, output_dtype=x.dtype)
        if mask is None:
            return output
        return torch.where(mask[:, :, None], output, torch.zeros_like(output))

    def extra_repr(self) -> str:
        config = self.config
        return (
            f"dim={config.dim}, num_heads={config.num_heads}, rank={config.rank}, "
            f"core_mode={config.core_mode.value}, "
            f"rank_rotary={config.rank_rotary}, eta=per-head-interior-tanh"
        )


__all__ = ["LSSO"]
