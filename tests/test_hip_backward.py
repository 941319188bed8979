"""First-order backward of the native mixer and module (GPU).

Bar (reference docs/CUDA_CONTRACT.md:93-101): finite gradients within rel L2
3e-2 of the FP64 reference.  Mixer-level gradients are checked against FP64
autograd through the ABI oracle (tests/cuda/test_fast_path.py:33-86 in the
reference); module-level gradients against the golden rank-48 vectors that
the real reference wrote (tests/golden/rank48_backward.npz).
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from lsso_amd import LSSO, LSSOConfig
from oracle import lsso_reference as oracle

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
GRAD_LIMIT = 3e-2


def _rel_l2(actual, expected) -> float:
    actual = torch.as_tensor(actual).detach().to(device="cpu", dtype=torch.float64)
    expected = torch.as_tensor(expected).detach().to(device="cpu", dtype=torch.float64)
    return float((actual - expected).norm() / expected.norm().clamp_min(1e-30))


def _inputs(batch, rank, heads, head_dim, length, seed, scale=0.05):
    generator = torch.Generator().manual_seed(seed)
    projected = torch.randn(batch, length, heads * (rank + head_dim), generator=generator).bfloat16()
    base = scale * torch.randn(heads, rank, rank, generator=generator)
    drive = scale * torch.randn(heads, head_dim, rank, generator=generator)
    eta_raw = 0.3 * torch.randn(heads, generator=generator)
    grad = torch.randn(batch, length, heads * head_dim, generator=generator).bfloat16()
    return projected, base, drive, eta_raw, grad


def _oracle_grads(projected, base, drive, eta_raw, grad, positions=None, counts=None):
    leaves = [projected.double().requires_grad_(), base.double().requires_grad_(),
              drive.double().requires_grad_(), eta_raw.double().requires_grad_()]
    out = oracle.fast_mix_fp64(*leaves, positions, counts)
    out.backward(grad.double())
    return [leaf.grad for leaf in leaves]


def _native_grads(native, projected, base, drive, eta_raw, grad, positions=None, counts=None):
    leaves = [projected.cuda().requires_grad_(), base.cuda().requires_grad_(),
              drive.cuda().requires_grad_(), eta_raw.cuda().requires_grad_()]
    out = native.fast_mix(*leaves, None if positions is None else positions.cuda(),
                          None if counts is None else counts.cuda())
    out.backward(grad.cuda())
    torch.cuda.synchronize()
    return [leaf.grad for leaf in leaves]


@pytest.mark.parametrize(
    ("batch", "rank", "heads", "head_dim", "length"),
    [
        (2, 16, 2, 16, 33),
        (2, 32, 2, 32, 100),
        (1, 48, 2, 32, 77),
        (1, 64, 1, 64, 65),
        (2, 32, 3, 17, 40),     # head_dim not a multiple of 16
        (1, 48, 2, 24, 129),
        (1, 32, 8, 32, 1024),
    ],
)
def test_mixer_gradients_match_fp64_autograd(native, batch, rank, heads, head_dim, length):
    projected, base, drive, eta_raw, grad = _inputs(batch, rank, heads, head_dim, length,
                                                    seed=500 + rank + head_dim + length)
    expected = _oracle_grads(projected, base, drive, eta_raw, grad)
    actual = _native_grads(native, projected, base, drive, eta_raw, grad)
    for name, a, e in zip(("projected", "core_base_raw", "core_drive_weight", "eta_raw"), actual, expected):
        assert a is not None and torch.isfinite(a).all(), name
        assert _rel_l2(a, e) <= GRAD_LIMIT, (name, _rel_l2(a, e))


def test_mixer_gradients_masked_per_sample_positions(native):
    batch, rank, heads, head_dim, length = 2, 32, 2, 32, 90
    projected, base, drive, eta_raw, grad = _inputs(batch, rank, heads, head_dim, length, seed=808)
    mask = torch.arange(length)[None, :] < torch.tensor([[90], [41]])
    projected = torch.where(mask[:, :, None], projected, torch.zeros_like(projected))
    grad = torch.where(mask[:, :, None], grad, torch.zeros_like(grad))
    position_ids = torch.stack((2 * torch.arange(length) + 5, torch.arange(length) + 300))
    positions = oracle.center_positions(position_ids, mask, dtype=torch.float32, all_valid=False)
    counts = mask.sum(dim=-1).float()
    expected = _oracle_grads(projected, base, drive, eta_raw, grad, positions, counts)
    actual = _native_grads(native, projected, base, drive, eta_raw, grad, positions, counts)
    for name, a, e in zip(("projected", "core_base_raw", "core_drive_weight", "eta_raw"), actual, expected):
        assert torch.isfinite(a).all(), name
        assert _rel_l2(a, e) <= GRAD_LIMIT, (name, _rel_l2(a, e))
    assert not actual[0].cpu()[~mask].any()


def test_zero_upstream_gives_zero_gradients(native):
    projected, base, drive, eta_raw, grad = _inputs(1, 32, 2, 32, 50, seed=9)
    actual = _native_grads(native, projected, base, drive, eta_raw, torch.zeros_like(grad))
    for value in actual:
        assert not value.any()


def test_mixer_backward_is_deterministic(native):
    projected, base, drive, eta_raw, grad = _inputs(2, 48, 2, 32, 300, seed=21)
    first = _native_grads(native, projected, base, drive, eta_raw, grad)
    second = _native_grads(native, projected, base, drive, eta_raw, grad)
    for a, b in zip(first, second):
        assert torch.equal(a, b)


def test_module_rank48_gradients_match_reference_golden(native):
    """C5-shaped check (rank 48, loss = mean(y^2)) at the golden case's size."""

    data = np.load(GOLDEN / "rank48_backward.npz")
    config = LSSOConfig(dim=96, num_heads=2, rank=48, bias=True)
    layer = LSSO(config).cuda()
    with torch.no_grad():
        for name, parameter in layer.named_parameters():
            parameter.copy_(torch.from_numpy(data[f"param:{name}"]))
    x = torch.from_numpy(data["x"]).half().cuda().requires_grad_()
    y = layer(x, implementation="hip")
    y.float().square().mean().backward()
    torch.cuda.synchronize()
    assert _rel_l2(y, data["y64"]) <= 5e-3
    assert _rel_l2(x.grad, data["grad64:x"]) <= GRAD_LIMIT
    for name, parameter in layer.named_parameters():
        assert parameter.grad is not None, name
        assert torch.isfinite(parameter.grad).all(), name
        assert _rel_l2(parameter.grad, data[f"grad64:{name}"]) <= GRAD_LIMIT, (name, _rel_l2(parameter.grad, data[f"grad64:{name}"]))


def test_module_backward_matches_oracle_autograd_masked(native):
    torch.manual_seed(5)
    config = LSSOConfig(dim=128, num_heads=4, rank=32, bias=True)
    layer = LSSO(config).cuda()
    with torch.no_grad():
        layer.core_base_raw.normal_(std=0.05)
        layer.core_drive_weight.normal_(std=0.05)
    x = torch.randn(2, 70, 128, generator=torch.Generator().manual_seed(6)).bfloat16().cuda().requires_grad_()
    mask = (torch.arange(70)[None, :] < torch.tensor([[70], [33]])).cuda()
    y = layer(x, valid_mask=mask, implementation="hip")
    y.float().square().mean().backward()
    params = {name: p.detach().double().cpu().requires_grad_() for name, p in layer.named_parameters()}
    x64 = x.detach().double().cpu().requires_grad_()
    expected = oracle.lsso_forward(params, {"dim": 128, "num_heads": 4, "rank": 32, "bias": True},
                                   x64, valid_mask=mask.cpu())
    expected.square().mean().backward()
    assert _rel_l2(x.grad, x64.grad) <= GRAD_LIMIT
    for name, parameter in layer.named_parameters():
        assert _rel_l2(parameter.grad, params[name].grad) <= GRAD_LIMIT, (name, _rel_l2(parameter.grad, params[name].grad))


@pytest.mark.parametrize(
    ("batch", "rank", "heads", "head_dim", "length"),
    [
        (2, 48, 8, 32, 300),   # resident token map: sums from its output tiles
        (2, 32, 2, 64, 129),   # resident, four content blocks
        (1, 16, 3, 24, 77),    # general token map: one pass over grad_projected
    ],
)
def test_backward_column_sums_match_grad_projected(native, batch, rank, heads, head_dim, length):
    projected, base, drive, eta_raw, grad = _inputs(batch, rank, heads, head_dim, length, seed=rank + length)
    args = [t.cuda() for t in (grad, projected, base, drive, eta_raw)]
    with torch.no_grad():
        _, tape = native.forward_train(args[1], args[2], args[3], args[4])
        plain = native.backward(*args, tape)
        *grads, sums = native.backward(*args, tape, column_sums=True)
    for a, b in zip(plain, grads):
        assert torch.equal(a, b)
    expected = grads[0].double().sum(dim=(0, 1))
    torch.testing.assert_close(sums.double(), expected, rtol=1e-5, atol=1e-4)


@pytest.mark.parametrize(("dim", "heads", "rank"), [(256, 2, 32), (192, 1, 64)])
def test_module_wide_head_gradients_match_oracle_autograd(native, dim, heads, rank):
    """head_dim 128 and 192: the panel-looped compact VJP and token map."""

    torch.manual_seed(17 + dim)
    config = LSSOConfig(dim=dim, num_heads=heads, rank=rank, bias=True)
    layer = LSSO(config).cuda()
    with torch.no_grad():
        layer.core_base_raw.normal_(std=0.05)
        layer.core_drive_weight.normal_(std=0.05)
    x = torch.randn(2, 150, dim, generator=torch.Generator().manual_seed(18)).half().cuda().requires_grad_()
    upstream = torch.randn(2, 150, dim, generator=torch.Generator().manual_seed(19))
    y = layer(x, implementation="hip")
    (y.float() * upstream.cuda()).sum().backward()
    params = {name: p.detach().double().cpu().requires_grad_() for name, p in layer.named_parameters()}
    x64 = x.detach().double().cpu().requires_grad_()
    expected = oracle.lsso_forward(params, {"dim": dim, "num_heads": heads, "rank": rank, "bias": True}, x64)
    (expected * upstream.double()).sum().backward()
    assert _rel_l2(y, expected) <= 5e-3
    assert _rel_l2(x.grad, x64.grad) <= GRAD_LIMIT
    for name, parameter in layer.named_parameters():
        assert _rel_l2(parameter.grad, params[name].grad) <= GRAD_LIMIT, (name, _rel_l2(parameter.grad, params[name].grad))


def test_module_d768_contract_shape_forward_backward(native, parity_report):
    """The reference's own exploratory contract-8 measurement shape
    (docs/CUDA_CONTRACT.md:270-275): B=2, N=4096, D=768, H=12, r=48, FP16.
    Both projections have in_features 768 and the input projection's value
    gradient 1,344, past the register-resident tiers: the K-streaming tier."""

    torch.manual_seed(768)
    config = LSSOConfig(dim=768, num_heads=12, rank=48, bias=True)
    layer = LSSO(config).cuda()
    with torch.no_grad():
        layer.core_base_raw.normal_(std=0.05)
        layer.core_drive_weight.normal_(std=0.05)
    x = torch.randn(2, 4096, 768, generator=torch.Generator().manual_seed(769)).half()
    upstream = torch.randn(2, 4096, 768, generator=torch.Generator().manual_seed(770))
    xd = x.cuda().requires_grad_()
    y = layer(xd, implementation="hip")
    (y.float() * upstream.cuda()).sum().backward()
    torch.cuda.synchronize()
    params = {name: p.detach().double().cpu().requires_grad_() for name, p in layer.named_parameters()}
    x64 = x.double().requires_grad_()
    cfg = {"dim": 768, "num_heads": 12, "rank": 48, "bias": True}
    expected = oracle.lsso_forward(params, cfg, x64)
    (expected * upstream.double()).sum().backward()
    fp32 = oracle.lsso_forward({n: p.detach().float() for n, p in params.items()}, cfg, x.float())
    parity_report.record("D768 H12 r48 B2 L4096 fp16 forward", y, fp32, expected.detach())
    pairs = {"x": (xd.grad, x64.grad)}
    pairs.update({name: (p.grad, params[name].grad) for name, p in layer.named_parameters()})
    errors = parity_report.record_grads("D768 H12 r48 B2 L4096 fp16 backward", pairs)
    assert _rel_l2(y, expected) <= 5e-3
    for name, error in errors.items():
        assert error <= GRAD_LIMIT, (name, error)
