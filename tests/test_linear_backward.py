"""Backward of the native biased projection (GPU).

The reference VJP (lsso/ball/reference.py:205-247): the upstream gradient is
rounded to BF16 for the value and weight gradients (BF16 operands, FP32
accumulation), and summed in FP32 over all rows for the bias gradient.  The
native upstream-gradient pass must give the BF16 copy bit for bit (round to
nearest even, as torch's conversion) with excluded rows zero, and column sums
equal to an FP64 sum within FP32 summation error; the module-level VJP is
checked against a torch statement of the reference's.
"""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


def _expected(g: torch.Tensor, mask: torch.Tensor | None):
    kept = g if mask is None else torch.where(mask[:, None], g, torch.zeros_like(g))
    return kept.to(torch.bfloat16), kept.double().sum(dim=0)


@pytest.mark.parametrize(
    ("rows", "cols", "dtype", "masked", "stride_pad"),
    [
        (131, 256, torch.float16, False, 0),
        (4099, 640, torch.bfloat16, True, 0),
        (2048, 256, torch.float16, True, 0),
        (77, 24, torch.bfloat16, False, 0),
        (300, 52, torch.float16, True, 3),
        (1, 8, torch.float16, False, 0),
        (5000, 1000, torch.float16, False, 8),
    ],
)
def test_grad_columns_copy_and_sums(native, rows, cols, dtype, masked, stride_pad) -> None:
    generator = torch.Generator(device="cuda").manual_seed(rows * 7 + cols)
    storage = torch.randn(rows, cols + stride_pad, device="cuda", generator=generator) * 3
    g = storage.to(dtype)[:, :cols]
    mask = None
    if masked:
        mask = torch.rand(rows, device="cuda", generator=generator) > 0.3
        g[~mask] = float("nan")  # excluded rows count as zero whatever they hold
    copy, sums = native._grad_columns(g, mask, True, True)
    expected_copy, expected_sums = _expected(g, mask)
    assert torch.equal(copy.view(torch.int16), expected_copy.view(torch.int16))
    scale = g.float().abs().nan_to_num(0.0).sum(dim=0).double()
    error = (sums.double() - expected_sums).abs()
    assert torch.all(error <= 1e-6 * scale + 1e-6), float((error - 1e-6 * scale).max())


def test_grad_columns_outputs_are_optional_and_deterministic(native) -> None:
    g = torch.randn(8192, 640, device="cuda").bfloat16()
    _, first = native._grad_columns(g, None, False, True)
    copy, second = native._grad_columns(g, None, True, True)
    assert torch.equal(first, second)
    assert torch.equal(copy, g)
    only_copy, none = native._grad_columns(g.half(), None, True, False)
    assert none is None and torch.equal(only_copy, g.half().bfloat16())


def test_grad_columns_without_rows_sums_to_zero(native) -> None:
    g = torch.empty(0, 40, device="cuda", dtype=torch.float16)
    copy, sums = native._grad_columns(g, None, True, True)
    assert copy.shape == (0, 40)
    assert torch.equal(sums, torch.zeros(40, device="cuda"))


def _reference_vjp(value, weight, grad, mask):
    """The reference VJP in torch: BF16 operands, FP32 accumulation."""

    if mask is not None:
        grad = torch.where(mask[..., None], grad, torch.zeros_like(grad))
    flat_grad = grad.reshape(-1, weight.shape[0])
    g16 = flat_grad.to(torch.bfloat16).float()
    flat_value = value.reshape(-1, weight.shape[1])
    if mask is not None:
        flat_value = torch.where(mask.reshape(-1, 1), flat_value, torch.zeros_like(flat_value))
    d_value = (g16 @ weight.to(torch.bfloat16).float()).to(value.dtype).reshape(value.shape)
    d_weight = g16.T @ flat_value.to(torch.bfloat16).float()
    d_bias = flat_grad.float().sum(dim=0)
    return d_value, d_weight, d_bias


@pytest.mark.parametrize(
    ("batch", "length", "in_features", "out_features", "dtype", "masked"),
    [
        (4, 512, 256, 640, torch.float16, False),
        (2, 300, 256, 256, torch.float16, True),
        (3, 129, 96, 144, torch.bfloat16, True),
        (2, 64, 512, 512, torch.bfloat16, False),
    ],
)
def test_projection_vjp_matches_reference_statement(
    native, batch, length, in_features, out_features, dtype, masked
) -> None:
    generator = torch.Generator(device="cuda").manual_seed(batch * length + in_features)
    value = torch.randn(batch, length, in_features, device="cuda", generator=generator).to(dtype)
    bound = in_features ** -0.5
    weight = ((torch.rand(out_features, in_features, device="cuda", generator=generator) * 2 - 1) * bound)
    bias = (torch.rand(out_features, device="cuda", generator=generator) * 2 - 1) * bound
    mask = (torch.rand(batch, length, device="cuda", generator=generator) > 0.25) if masked else None
    if mask is not None:
        value[~mask] = float("nan")
    grad = torch.randn(batch, length, out_features, device="cuda", generator=generator).to(dtype)
    value.requires_grad_(True)
    weight.requires_grad_(True)
    bias.requires_grad_(True)
    out = native.linear(value, weight, bias, dtype, row_mask=mask)
    out.backward(grad)
    d_value, d_weight, d_bias = _reference_vjp(value.detach(), weight.detach(), grad, mask)
    if mask is not None:
        assert torch.count_nonzero(value.grad[~mask]) == 0
        got_value, want_value = value.grad[mask], d_value[mask]
    else:
        got_value, want_value = value.grad, d_value
    torch.testing.assert_close(got_value, want_value, rtol=torch.finfo(dtype).eps, atol=1e-5)
    torch.testing.assert_close(weight.grad, d_weight, rtol=1e-4, atol=1e-3)
    torch.testing.assert_close(bias.grad, d_bias, rtol=1e-5, atol=1e-4)


def test_projection_vjp_of_a_broadcast_upstream_gradient(native) -> None:
    """loss = y.sum(dim=(0, 1)) . v hands the projection an upstream gradient
    whose row strides are 0; the native VJP must see it as the dense tensor
    it stands for."""

    generator = torch.Generator(device="cuda").manual_seed(31)
    value = torch.randn(3, 70, 64, device="cuda", generator=generator).half().requires_grad_(True)
    weight = (0.1 * torch.randn(48, 64, device="cuda", generator=generator)).requires_grad_(True)
    bias = torch.randn(48, device="cuda", generator=generator).requires_grad_(True)
    direction = torch.randn(48, device="cuda", generator=generator)
    out = native.linear(value, weight, bias, torch.float16)
    (out.sum(dim=(0, 1)).float() * direction).sum().backward()
    dense = direction.half().expand(3, 70, 48).contiguous()
    d_value, d_weight, d_bias = _reference_vjp(value.detach(), weight.detach(), dense, None)
    torch.testing.assert_close(value.grad, d_value, rtol=torch.finfo(torch.float16).eps, atol=1e-5)
    torch.testing.assert_close(weight.grad, d_weight, rtol=1e-4, atol=1e-3)
    torch.testing.assert_close(bias.grad, d_bias, rtol=1e-5, atol=1e-4)


def test_module_trains_with_a_summed_loss_and_runs_on_expanded_x(native) -> None:
    from lsso_amd import LSSO, LSSOConfig
    from oracle import lsso_reference as oracle

    torch.manual_seed(7)
    layer = LSSO(LSSOConfig(dim=64, num_heads=2, rank=16, bias=True)).cuda()
    base = torch.randn(1, 40, 64, generator=torch.Generator().manual_seed(8)).half()
    expanded = base.cuda().expand(3, 40, 64)
    with torch.no_grad():
        out_expanded = layer(expanded, implementation="hip")
        out_dense = layer(expanded.contiguous(), implementation="hip")
    assert torch.equal(out_expanded, out_dense)

    x = expanded.contiguous().requires_grad_(True)
    direction = torch.randn(64, generator=torch.Generator().manual_seed(9))
    y = layer(x, implementation="hip")
    (y.float().sum(dim=(0, 1)) * direction.cuda()).sum().backward()
    params = {name: p.detach().double().cpu().requires_grad_() for name, p in layer.named_parameters()}
    x64 = x.detach().double().cpu().requires_grad_()
    y64 = oracle.lsso_forward(params, {"dim": 64, "num_heads": 2, "rank": 16, "bias": True}, x64)
    (y64.sum(dim=(0, 1)) * direction.double()).sum().backward()

    def rel(a, e):
        a = a.detach().double().cpu()
        return float((a - e).norm() / e.norm())

    assert rel(x.grad, x64.grad) <= 3e-2
    for name, parameter in layer.named_parameters():
        assert rel(parameter.grad, params[name].grad) <= 3e-2, name


@pytest.mark.parametrize(
    ("rows", "in_features", "out_features", "g_dtype", "x_dtype", "masked", "pad"),
    [
        (131072, 256, 640, torch.bfloat16, torch.float16, False, 0),   # C5 input projection
        (131072, 256, 256, torch.float16, torch.bfloat16, False, 0),   # C5 output projection
        (8192, 768, 1344, torch.bfloat16, torch.float16, True, 0),     # D = 768 input projection
        (4099, 200, 72, torch.float16, torch.float16, True, 8),        # strided rows, partial tiles
        (777, 41, 13, torch.bfloat16, torch.float16, False, 3),        # scalar loads (odd widths)
        (31, 64, 48, torch.float16, torch.float16, True, 0),           # fewer rows than one stage
        (320, 4096, 4096, torch.bfloat16, torch.bfloat16, False, 0),   # 1,024 output tiles: one split
    ],
)
def test_weight_gradient_kernel_matches_fp64_of_bf16_operands(
    native, rows, in_features, out_features, g_dtype, x_dtype, masked, pad
) -> None:
    generator = torch.Generator(device="cuda").manual_seed(rows + in_features + out_features)
    g = (torch.randn(rows, out_features + pad, device="cuda", generator=generator)).to(g_dtype)[:, :out_features]
    x = (torch.randn(rows, in_features + pad, device="cuda", generator=generator)).to(x_dtype)[:, :in_features]
    mask = None
    if masked:
        mask = torch.rand(rows, device="cuda", generator=generator) > 0.3
        g = g.clone()
        x = x.clone()
        g[~mask] = float("nan")   # excluded rows count as zero whatever they hold
        x[~mask] = float("nan")
    grad_weight, grad_bias = native._weight_gradient(g, x, mask, True)
    keep = torch.ones(rows, dtype=torch.bool, device="cuda") if mask is None else mask
    g64 = torch.where(keep[:, None], g.to(torch.bfloat16).double(), 0.0)
    x64 = torch.where(keep[:, None], x.to(torch.bfloat16).double(), 0.0)
    expected = g64.T @ x64
    scale = g64.abs().T @ x64.abs()
    error = (grad_weight.double() - expected).abs()
    # FP32 accumulation: chains of at most a few thousand terms per split.
    assert torch.all(error <= 1e-5 * scale + 1e-6), float((error / (scale + 1e-30)).max())
    sums64 = torch.where(keep[:, None], g.double(), 0.0).sum(dim=0)
    sum_scale = torch.where(keep[:, None], g.double().abs(), 0.0).sum(dim=0)
    assert torch.all((grad_bias.double() - sums64).abs() <= 1e-6 * sum_scale + 1e-6)
    again, again_bias = native._weight_gradient(g, x, mask, True)
    assert torch.equal(again, grad_weight) and torch.equal(again_bias, grad_bias)


def test_weight_gradient_of_no_rows_is_zero(native) -> None:
    g = torch.empty(0, 24, device="cuda", dtype=torch.float16)
    x = torch.empty(0, 40, device="cuda", dtype=torch.bfloat16)
    grad_weight, grad_bias = native._weight_gradient(g, x, None, True)
    assert torch.equal(grad_weight, torch.zeros(24, 40, device="cuda"))
    assert torch.equal(grad_bias, torch.zeros(24, device="cuda"))
