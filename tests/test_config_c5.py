"""Config C5 end to end on the GPU: forward + first-order backward of the
complete mixer at its full size (B=64, N=2048, D=256, H=8, r=48, FP16 x,
loss = mean(y.float()^2)), checked against FP64 autograd through the CPU
oracle.  Mirrors the reference's module gradient check
(tests/cuda/test_fast_path.py:1316-1370) at the benchmark shape.

The oracle's gradients are sums over 8-sample slices of the batch, each
slice's loss normalised by the full batch's element count, so they are the
full-batch gradients (the loss is a sum over samples).

FP16 training scales the loss.  The gradient that autograd hands to the FP16
output y is stored in FP16, and d mean(y^2) / dy = 2 y / N with N = 33.5 M
elements is about 6e-8, below FP16's smallest normal number (6.1e-5): it
would reach the mixer as subnormal or zero values.  The native path is
therefore run on LOSS_SCALE * mean(y^2), the initial scale of
torch.amp.GradScaler, and its gradients are divided by LOSS_SCALE before the
comparison, as GradScaler.unscale_ does."""

from __future__ import annotations

import pytest
import torch

from lsso_amd import LSSO, LSSOConfig
from oracle import lsso_reference as oracle

pytestmark = pytest.mark.gpu

FORWARD_LIMIT = 5e-3
GRAD_LIMIT = 3e-2
LOSS_SCALE = 2.0 ** 16


def _rel_l2(actual, expected) -> float:
    actual = torch.as_tensor(actual).detach().to(device="cpu", dtype=torch.float64)
    expected = torch.as_tensor(expected).detach().to(device="cpu", dtype=torch.float64)
    return float((actual - expected).norm() / expected.norm().clamp_min(1e-300))


def test_config_c5_forward_backward_matches_fp64_oracle(native, parity_report) -> None:
    batch, length, dim, heads, rank = 64, 2048, 256, 8, 48
    torch.manual_seed(0)
    config = LSSOConfig(dim=dim, num_heads=heads, rank=rank, bias=True)
    layer = LSSO(config)
    with torch.no_grad():
        layer.core_base_raw.normal_(std=0.05)
        layer.core_drive_weight.normal_(std=0.05)
    layer = layer.cuda().train()
    x = torch.randn(batch, length, dim, generator=torch.Generator().manual_seed(1)).half()
    xd = x.cuda().requires_grad_()
    y = layer(xd, implementation="hip")
    (LOSS_SCALE * y.float().square().mean()).backward()
    torch.cuda.synchronize()
    assert torch.isfinite(y).all()
    assert torch.isfinite(xd.grad).all()
    for name, parameter in layer.named_parameters():
        assert parameter.grad is not None and torch.isfinite(parameter.grad).all(), name

    picks = [0, 31, 63]
    cfg = {"dim": dim, "num_heads": heads, "rank": rank, "bias": True}
    params = {name: p.detach().double().cpu().requires_grad_() for name, p in layer.named_parameters()}
    elements = batch * length * dim
    y64 = {}
    gx64 = {}
    for start in range(0, batch, 8):
        xs = x[start:start + 8].double().requires_grad_()
        ys = oracle.lsso_forward(params, cfg, xs)
        (ys.square().sum() / elements).backward()
        for pick in picks:
            if start <= pick < start + 8:
                y64[pick] = ys[pick - start].detach()
                gx64[pick] = xs.grad[pick - start]
    expected_y = torch.stack([y64[p] for p in picks])
    expected_gx = torch.stack([gx64[p] for p in picks])
    params32 = {name: p.detach().float().cpu() for name, p in layer.named_parameters()}
    fp32 = oracle.lsso_forward(params32, cfg, x[picks].float())

    parity_report.record("C5 B64 D256 H8 r48 L2048 fp16 forward (samples 0,31,63)", y[picks], fp32,
                         expected_y)
    pairs = {"x(0,31,63)": (xd.grad[picks].float() / LOSS_SCALE, expected_gx)}
    pairs.update({name: (p.grad / LOSS_SCALE, params[name].grad) for name, p in layer.named_parameters()})
    errors = parity_report.record_grads("C5 B64 D256 H8 r48 L2048 fp16 backward", pairs)
    assert _rel_l2(y[picks], expected_y) <= FORWARD_LIMIT
    for name, error in errors.items():
        assert error <= GRAD_LIMIT, (name, error)
