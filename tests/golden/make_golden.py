"""Write the golden fixtures that pin the CPU oracle to the real reference.

Run once, in the build container where the reference tree is mounted:

    python tests/golden/make_golden.py /root/reference

It imports the reference package ``lsso`` (CPU only, no native code) and
records inputs and outputs of its public forward for a few small cases.  The
fixtures hold data only (inputs, parameters, outputs); no reference source is
copied.  Closed forms pin the mathematics in FP64; these vectors additionally
pin what closed forms leave open: the exact FP32 operation order and the
BF16/FP16 rounding boundaries of the reference CPU path, the default-init
state_dict under a seed, and the ABI-level FP64 composition of the native
tests (tests/cuda/test_fast_path.py:33-86 in the reference).
"""

from __future__ import annotations

import copy
from pathlib import Path
import sys

import numpy as np
import torch

HERE = Path(__file__).resolve().parent


def _np(value: torch.Tensor) -> np.ndarray:
    value = value.detach()
    if value.dtype == torch.bfloat16:
        value = value.to(torch.float32)
    return value.cpu().numpy()


def _state(layer) -> dict[str, np.ndarray]:
    return {
        f"param:{name}": _np(parameter) for name, parameter in layer.named_parameters()
    }


def main(reference_root: str) -> None:
    sys.path.insert(0, reference_root)
    import lsso  # noqa: E402
    from lsso import LSSO, LSSOConfig  # noqa: E402
    from lsso.ball import reference as ref  # noqa: E402

    torch.set_num_threads(1)

    # C1: default-init DYNAMIC + Rank-Rotary, shared positions, no mask.
    torch.manual_seed(0)
    layer = LSSO(LSSOConfig(dim=192, num_heads=3, rank=16)).eval()
    x = torch.randn(8, 65, 192, generator=torch.Generator().manual_seed(1))
    with torch.no_grad():
        y32 = layer(x)
        projected, frame, compact_state, _content, generator, eta, _mask = (
            layer._reference_compact_problem(x, None, None)
        )
        layer64 = copy.deepcopy(layer).double()
        y64 = layer64(x.double())
    np.savez_compressed(
        HERE / "c1_default.npz",
        reference_version=np.array(lsso.__version__),
        x=_np(x),
        y32=_np(y32),
        y64=_np(y64),
        projected=_np(projected),
        frame=_np(frame),
        compact_state=_np(compact_state),
        generator=_np(generator),
        eta=_np(eta),
        **_state(layer),
    )

    # Masked (gapped + trailing padding, one all-masked row), per-sample
    # integer positions, biased projections, non-zero compact core.
    torch.manual_seed(5)
    layer = LSSO(LSSOConfig(dim=24, num_heads=2, rank=8, bias=True)).eval()
    with torch.no_grad():
        layer.core_base_raw.normal_(std=0.1)
        layer.core_drive_weight.normal_(std=0.1)
        layer.eta_raw.normal_(std=0.3)
    mask = torch.tensor(
        [
            [True, False, True, True, False, True, True, True, False, True, False, False],
            [False, True, True, True, True, True, True, False, True, True, True, True],
            [False] * 12,
        ]
    )
    clean = torch.randn(3, 12, 24, generator=torch.Generator().manual_seed(6))
    x = torch.where(mask[:, :, None], clean, torch.full_like(clean, float("nan")))
    positions = torch.stack(
        (3 * torch.arange(12) + 11, 5 * torch.arange(12) + 101, torch.arange(12))
    )
    with torch.no_grad():
        y32 = layer(x, valid_mask=mask, position_ids=positions)
        y64 = copy.deepcopy(layer).double()(x.double(), valid_mask=mask, position_ids=positions)
    np.savez_compressed(
        HERE / "masked.npz",
        x=_np(x),
        mask=mask.numpy(),
        position_ids=positions.numpy(),
        y32=_np(y32),
        y64=_np(y64),
        **_state(layer),
    )

    # Rank 48 (non-power-of-two) with gradients of mean(y^2).
    torch.manual_seed(48)
    layer = LSSO(LSSOConfig(dim=96, num_heads=2, rank=48, bias=True))
    with torch.no_grad():
        layer.core_base_raw.normal_(std=0.05)
        layer.core_drive_weight.normal_(std=0.05)
    x = torch.randn(2, 20, 96, generator=torch.Generator().manual_seed(49))
    grads = {}
    for tag, module, value in (
        ("32", layer, x.clone().requires_grad_()),
        ("64", copy.deepcopy(layer).double(), x.double().requires_grad_()),
    ):
        module.zero_grad(set_to_none=True)
        y = module(value)
        y.square().mean().backward()
        grads[f"y{tag}"] = _np(y)
        grads[f"grad{tag}:x"] = _np(value.grad)
        for name, parameter in module.named_parameters():
            grads[f"grad{tag}:{name}"] = _np(parameter.grad)
    np.savez_compressed(HERE / "rank48_backward.npz", x=_np(x), **_state(layer), **grads)

    # ABI-level FP64 oracle of the native mixer (reference tests/cuda/
    # test_fast_path.py:33-86), composed from the reference's functions.
    def fast_mix64(projected, base, drive, eta_raw, positions, counts):
        projected = projected.double()
        base = base.double()
        drive = drive.double()
        batch, length, width = projected.shape
        heads, rank = base.shape[0], base.shape[-1]
        dim = width - heads * rank
        relation, content = projected.split((heads * rank, dim), dim=-1)
        relation = relation.view(batch, length, heads, rank).transpose(1, 2)
        content = content.view(batch, length, heads, dim // heads).transpose(1, 2)
        counts64 = counts.double()
        relation = ref.rank_rotary(relation, positions.double().expand(batch, -1)) / counts64.sqrt().view(batch, 1, 1, 1)
        frame = ref.qr_soft_frame(relation)
        compact = frame.mT @ content
        coordinates = base.unsqueeze(0) + compact @ drive / counts64.sqrt().view(batch, 1, 1, 1)
        return ref.accretive_equilibrium_mix(
            frame, ref.accretive_generator(coordinates), compact, content,
            ref.bounded_complement(eta_raw.double()),
        ).transpose(1, 2).contiguous().view(batch, length, dim)

    generator_ = torch.Generator().manual_seed(33)
    cases = {}
    for tag, (batch, rank, heads, head_dim, length) in {
        "r32": (2, 32, 2, 17, 33),
        "r48": (1, 48, 2, 24, 40),
    }.items():
        projected = torch.randn(batch, length, heads * (rank + head_dim), generator=generator_).bfloat16()
        base = 0.1 * torch.randn(heads, rank, rank, generator=generator_)
        drive = 0.1 * torch.randn(heads, head_dim, rank, generator=generator_)
        eta_raw = 0.3 * torch.randn(heads, generator=generator_)
        positions = torch.arange(length, dtype=torch.float64) - 0.5 * (length - 1)
        counts = torch.full((batch,), float(length))
        out = fast_mix64(projected, base, drive, eta_raw, positions, counts)
        cases.update({
            f"{tag}:projected": _np(projected), f"{tag}:base": _np(base),
            f"{tag}:drive": _np(drive), f"{tag}:eta_raw": _np(eta_raw),
            f"{tag}:mixed64": _np(out),
        })
    np.savez_compressed(HERE / "fast_mix.npz", **cases)
    for path in sorted(HERE.glob("*.npz")):
        print(path.name, path.stat().st_size)


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
