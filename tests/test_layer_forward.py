"""The whole-layer native forward against the three-call native path (GPU).

``lsso_hip_layer_forward`` runs the input projection fused with the token
reductions (the packed tile is reduced in LDS, not read back) and the apply
fused with the output projection.  The reductions run the same MFMA chains
over the same token chunks as ``reduce_kernel`` and the projection the same
K order and rounding as ``linear_kernel``, so the result must equal
``linear -> forward_inference -> linear`` bit for bit.  Parity of that path
with the FP64 oracle is tested in tests/test_hip_parity.py; one direct oracle
check is kept here as well.
"""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


def _layer_inputs(batch, rank, heads, head_dim, length, seed, dtype=torch.float16, scale=0.05):
    generator = torch.Generator().manual_seed(seed)
    dim = heads * head_dim
    width = heads * rank + dim
    x = torch.randn(batch, length, dim, generator=generator).to(dtype)
    in_weight = torch.randn(width, dim, generator=generator) / dim**0.5
    in_bias = 0.1 * torch.randn(width, generator=generator)
    base = scale * torch.randn(heads, rank, rank, generator=generator)
    drive = scale * torch.randn(heads, head_dim, rank, generator=generator)
    eta_raw = scale * torch.randn(heads, generator=generator)
    out_weight = torch.randn(dim, dim, generator=generator) / dim**0.5
    out_bias = 0.1 * torch.randn(dim, generator=generator)
    return [t.cuda() for t in (x, in_weight, in_bias, base, drive, eta_raw, out_weight, out_bias)]


def _three_calls(native, x, in_weight, in_bias, base, drive, eta_raw, positions, counts,
                 out_weight, out_bias, mask):
    projected = native.linear(x, in_weight, in_bias, torch.bfloat16, row_mask=mask)
    mixed = native.forward_inference(projected, base, drive, eta_raw, positions, counts)
    return native.linear(mixed, out_weight, out_bias, x.dtype, row_mask=mask)


@pytest.mark.parametrize(
    ("batch", "rank", "heads", "head_dim", "length"),
    [
        (2, 32, 8, 32, 1000),   # headline geometry: 2 head groups, ragged tail tile
        (2, 32, 8, 32, 4096),   # headline length: 4 chunks of 1024 tokens
        (2, 48, 8, 32, 333),    # C5 geometry: 3 head groups, the last with 2 heads
        (1, 64, 6, 64, 300),    # C4 geometry: D = 384 (4-wave tier), unfused output side
        (3, 16, 8, 16, 65),     # D = 128, rank 16 (one pair slot per lane)
        (2, 16, 3, 64, 37),     # C1 geometry, shorter than one tile
        (1, 48, 2, 64, 130),    # rank 48 with 64-feature heads (two content blocks)
    ],
)
@pytest.mark.parametrize("dtype", (torch.float16, torch.bfloat16))
def test_layer_forward_is_bitwise_the_three_call_path(native, batch, rank, heads, head_dim, length, dtype):
    x, in_w, in_b, base, drive, eta_raw, out_w, out_b = _layer_inputs(
        batch, rank, heads, head_dim, length, seed=3000 + rank + head_dim + length, dtype=dtype
    )
    with torch.no_grad():
        assert native.layer_supported(x, in_w, base, drive, eta_raw)
        y = native.layer_forward(x, in_w, in_b, base, drive, eta_raw, None, None, out_w, out_b)
        expected = _three_calls(native, x, in_w, in_b, base, drive, eta_raw, None, None, out_w, out_b, None)
    torch.cuda.synchronize()
    assert y.dtype == dtype
    assert torch.isfinite(y).all()
    assert torch.equal(y, expected)


def test_layer_forward_masked_per_sample_positions_and_no_bias(native):
    batch, rank, heads, head_dim, length = 3, 32, 8, 32, 700
    x, in_w, _in_b, base, drive, eta_raw, out_w, _out_b = _layer_inputs(
        batch, rank, heads, head_dim, length, seed=91
    )
    lengths = torch.tensor([700, 123, 1])
    mask = (torch.arange(length)[None, :] < lengths[:, None]).cuda()
    # Garbage (NaN) in masked rows must not leak: masked rows project to zero.
    x = torch.where(mask[:, :, None], x, torch.full_like(x, float("nan")))
    positions = (torch.arange(length)[None, :] * torch.tensor([[1.0], [3.0], [7.0]])).cuda()
    positions = positions - positions.mean(dim=1, keepdim=True)
    counts = lengths.float().cuda()
    with torch.no_grad():
        y = native.layer_forward(x, in_w, None, base, drive, eta_raw, positions, counts, out_w, None,
                                 row_mask=mask)
        expected = _three_calls(native, x, in_w, None, base, drive, eta_raw, positions, counts, out_w,
                                None, mask)
    torch.cuda.synchronize()
    assert torch.isfinite(y).all()
    assert torch.equal(y, expected)
    assert not y[~mask].any()


def test_layer_forward_shared_positions(native):
    batch, rank, heads, head_dim, length = 2, 48, 8, 32, 200
    x, in_w, in_b, base, drive, eta_raw, out_w, out_b = _layer_inputs(
        batch, rank, heads, head_dim, length, seed=92
    )
    positions = (0.5 * torch.arange(length, dtype=torch.float32) - 20.0).cuda()
    positions = positions - positions.mean()
    with torch.no_grad():
        y = native.layer_forward(x, in_w, in_b, base, drive, eta_raw, positions, None, out_w, out_b)
        expected = _three_calls(native, x, in_w, in_b, base, drive, eta_raw, positions, None, out_w,
                                out_b, None)
    torch.cuda.synchronize()
    assert torch.equal(y, expected)


def test_layer_forward_rejects_unsupported_geometry_and_autograd(native):
    # D = 512 is past the fused projection's K tiers.
    x, in_w, in_b, base, drive, eta_raw, out_w, out_b = _layer_inputs(1, 32, 8, 64, 40, seed=7)
    with torch.no_grad():
        assert not native.layer_supported(x, in_w, base, drive, eta_raw)
        with pytest.raises(ValueError, match="fused layer"):
            native.layer_forward(x, in_w, in_b, base, drive, eta_raw, None, None, out_w, out_b)
    x, in_w, in_b, base, drive, eta_raw, out_w, out_b = _layer_inputs(1, 32, 4, 32, 40, seed=8)
    in_w.requires_grad_(True)
    with pytest.raises(RuntimeError, match="inference-only"):
        native.layer_forward(x, in_w, in_b, base, drive, eta_raw, None, None, out_w, out_b)


def test_module_runs_the_layer_path_and_matches_the_oracle(native):
    """Module inference goes through lsso_hip_layer_forward and stays within
    the reference envelope of the FP64 oracle (rel L2 <= 5e-3,
    docs/CUDA_CONTRACT.md:93-101 in the reference)."""

    from lsso_amd import LSSO, LSSOConfig
    from oracle import lsso_reference as oracle

    torch.manual_seed(11)
    layer = LSSO(LSSOConfig(dim=256, num_heads=8, rank=32, bias=True)).cuda().eval()
    with torch.no_grad():
        layer.core_base_raw.normal_(std=0.05)
        layer.core_drive_weight.normal_(std=0.05)
        layer.eta_raw.normal_(std=0.3)
    x = torch.randn(2, 300, 256, generator=torch.Generator().manual_seed(12)).half().cuda()
    calls = []
    original = native.layer_forward

    def spy(*args, **kwargs):
        calls.append(1)
        return original(*args, **kwargs)

    native.layer_forward = spy
    try:
        with torch.no_grad():
            y = layer(x, implementation="hip")
    finally:
        native.layer_forward = original
    torch.cuda.synchronize()
    assert calls, "module inference did not take the fused layer path"
    config = {"dim": 256, "num_heads": 8, "rank": 32, "bias": True}
    params = {name: p.detach().double().cpu() for name, p in layer.named_parameters()}
    expected = oracle.lsso_forward(params, config, x.cpu().double())
    got = y.detach().to(device="cpu", dtype=torch.float64)
    rel = float((got - expected).norm() / expected.norm())
    assert rel <= 5e-3, rel


# -- training forward: projection + mixer in one call -------------------------
@pytest.mark.parametrize(
    ("batch", "rank", "heads", "head_dim", "length", "masked"),
    [
        (2, 48, 8, 32, 333, False),   # C5 geometry
        (2, 32, 8, 32, 1000, True),
        (1, 64, 6, 64, 300, True),    # C4 geometry
        (3, 16, 8, 16, 65, False),
    ],
)
def test_project_mix_is_bitwise_linear_then_forward_train(native, batch, rank, heads, head_dim, length, masked):
    x, in_w, in_b, base, drive, eta_raw, _out_w, _out_b = _layer_inputs(
        batch, rank, heads, head_dim, length, seed=5000 + rank + length
    )
    positions, counts, mask = None, None, None
    if masked:
        generator = torch.Generator().manual_seed(length)
        valid = torch.randint(length // 4, length + 1, (batch,), generator=generator)
        mask = (torch.arange(length)[None, :] < valid[:, None]).cuda()
        counts = valid.float().cuda()
        starts = torch.randint(0, 1024, (batch, 1), generator=generator).float()
        raw = starts + torch.arange(length, dtype=torch.float32)[None, :]
        centre = (raw * mask.cpu()).sum(dim=1, keepdim=True) / valid[:, None]
        positions = (raw - centre).cuda()
    with torch.no_grad():
        assert native.layer_supported(x, in_w, base, drive, eta_raw)
        packed, mixed, tape = native._project_mix_forward(
            x, in_w, in_b, base, drive, eta_raw, positions, counts, mask, True
        )
        projected = native.linear(x, in_w, in_b, torch.bfloat16, row_mask=mask)
        expected_mixed, expected_tape = native.forward_train(projected, base, drive, eta_raw, positions, counts)
    torch.cuda.synchronize()
    assert torch.equal(packed, projected)
    assert torch.equal(mixed, expected_mixed)
    assert torch.equal(tape, expected_tape)


@pytest.mark.parametrize(
    ("mode", "batch", "rank", "heads", "head_dim", "length", "masked"),
    [
        ("1", 2, 48, 8, 32, 333, False),   # C5 geometry fused: 3 head groups, the last with 2 heads
        ("1", 1, 64, 6, 64, 300, True),    # C4 geometry fused: D = 384 (4-wave tier), masked
        ("1", 1, 48, 2, 64, 130, True),    # rank 48 with 64-feature heads (two content blocks)
        ("0", 2, 32, 8, 32, 1000, True),   # headline geometry with the separate kernels
    ],
)
def test_fused_projection_override_keeps_the_bits(native, monkeypatch, mode, batch, rank, heads, head_dim,
                                                  length, masked):
    """LSSO_HIP_FUSED_PROJECTION=1 runs the fused projection + reduce kernel at
    ranks where the library would otherwise run the projection and the reduce
    separately (and =0 the reverse); the layer forward and the training forward
    must still equal the separate calls bit for bit."""
    x, in_w, in_b, base, drive, eta_raw, out_w, out_b = _layer_inputs(
        batch, rank, heads, head_dim, length, seed=7000 + rank + length
    )
    positions, counts, mask = None, None, None
    if masked:
        generator = torch.Generator().manual_seed(length + 1)
        valid = torch.randint(length // 4, length + 1, (batch,), generator=generator)
        mask = (torch.arange(length)[None, :] < valid[:, None]).cuda()
        counts = valid.float().cuda()
        starts = torch.randint(0, 1024, (batch, 1), generator=generator).float()
        raw = starts + torch.arange(length, dtype=torch.float32)[None, :]
        centre = (raw * mask.cpu()).sum(dim=1, keepdim=True) / valid[:, None]
        positions = (raw - centre).cuda()
    with torch.no_grad():
        expected = _three_calls(native, x, in_w, in_b, base, drive, eta_raw, positions, counts, out_w, out_b, mask)
        projected = native.linear(x, in_w, in_b, torch.bfloat16, row_mask=mask)
        expected_mixed, expected_tape = native.forward_train(projected, base, drive, eta_raw, positions, counts)
        monkeypatch.setenv("LSSO_HIP_FUSED_PROJECTION", mode)
        y = native.layer_forward(x, in_w, in_b, base, drive, eta_raw, positions, counts, out_w, out_b,
                                 row_mask=mask)
        packed, mixed, tape = native._project_mix_forward(
            x, in_w, in_b, base, drive, eta_raw, positions, counts, mask, True
        )
    torch.cuda.synchronize()
    assert torch.equal(y, expected)
    assert torch.equal(packed, projected)
    assert torch.equal(mixed, expected_mixed)
    assert torch.equal(tape, expected_tape)


def test_project_mix_gradients_equal_the_two_call_path(native):
    x, in_w, in_b, base, drive, eta_raw, out_w, out_b = _layer_inputs(2, 48, 8, 32, 300, seed=77)
    mask = torch.ones(2, 300, dtype=torch.bool, device="cuda")
    mask[1, 250:] = False
    counts = mask.sum(dim=1).float()
    positions = torch.arange(300, dtype=torch.float32, device="cuda")[None, :].repeat(2, 1)
    positions = positions - (positions * mask).sum(dim=1, keepdim=True) / counts[:, None]
    upstream = torch.randn(2, 300, 8 * 32, device="cuda").bfloat16()

    def run(fused: bool):
        leaves = [t.detach().clone().requires_grad_(True) for t in (x, in_w, in_b, base, drive, eta_raw)]
        if fused:
            mixed = native.project_mix(*leaves, positions, counts, row_mask=mask)
        else:
            projected = native.linear(leaves[0], leaves[1], leaves[2], torch.bfloat16, row_mask=mask)
            mixed = native.fast_mix(projected, leaves[3], leaves[4], leaves[5], positions, counts)
        mixed.backward(upstream)
        return mixed.detach(), [leaf.grad for leaf in leaves]

    fused_out, fused_grads = run(True)
    split_out, split_grads = run(False)
    assert torch.equal(fused_out, split_out)
    names = ("x", "in_weight", "in_bias", "base", "drive", "eta")
    for name, got, want in zip(names, fused_grads, split_grads):
        assert got is not None and torch.isfinite(got).all(), name
        if name == "in_bias":
            # Summed inside the token map: the same FP32 sums in another fixed order.
            torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-5)
        else:
            assert torch.equal(got, want), name


# -- training forward of the whole layer in one call --------------------------
@pytest.mark.parametrize(
    ("batch", "rank", "heads", "head_dim", "length", "masked"),
    [
        (2, 48, 8, 32, 333, False),   # C5 geometry: apply + output projection fused, 640-column rows
        (2, 32, 8, 32, 1000, True),
        (1, 64, 6, 64, 300, True),    # C4 geometry: D = 384, apply and projection separate
        (3, 16, 8, 16, 65, False),
    ],
)
def test_layer_train_is_bitwise_the_three_call_path(native, batch, rank, heads, head_dim, length, masked):
    x, in_w, in_b, base, drive, eta_raw, out_w, out_b = _layer_inputs(
        batch, rank, heads, head_dim, length, seed=6000 + rank + length
    )
    positions, counts, mask = None, None, None
    if masked:
        generator = torch.Generator().manual_seed(length + 1)
        valid = torch.randint(length // 4, length + 1, (batch,), generator=generator)
        mask = (torch.arange(length)[None, :] < valid[:, None]).cuda()
        counts = valid.float().cuda()
        raw = torch.arange(length, dtype=torch.float32)[None, :].repeat(batch, 1)
        centre = (raw * mask.cpu()).sum(dim=1, keepdim=True) / valid[:, None]
        positions = (raw - centre).cuda()
    with torch.no_grad():
        packed, mixed, tape, y = native._project_mix_forward(
            x, in_w, in_b, base, drive, eta_raw, positions, counts, mask, True, out_w, out_b
        )
        expected_packed, expected_mixed, expected_tape = native._project_mix_forward(
            x, in_w, in_b, base, drive, eta_raw, positions, counts, mask, True
        )
        expected_y = native.linear(expected_mixed, out_w, out_b, x.dtype, row_mask=mask)
    torch.cuda.synchronize()
    assert torch.equal(packed, expected_packed)
    assert torch.equal(mixed, expected_mixed)
    assert torch.equal(tape, expected_tape)
    assert torch.equal(y, expected_y)
    if mask is not None:
        assert not y[~mask].any()


def test_layer_train_gradients_equal_the_three_call_path(native):
    x, in_w, in_b, base, drive, eta_raw, out_w, out_b = _layer_inputs(2, 48, 8, 32, 300, seed=78)
    mask = torch.ones(2, 300, dtype=torch.bool, device="cuda")
    mask[1, 250:] = False
    counts = mask.sum(dim=1).float()
    positions = torch.arange(300, dtype=torch.float32, device="cuda")[None, :].repeat(2, 1)
    positions = positions - (positions * mask).sum(dim=1, keepdim=True) / counts[:, None]
    upstream = torch.randn(2, 300, 8 * 32, device="cuda").half()

    def run(fused: bool):
        leaves = [t.detach().clone().requires_grad_(True) for t in (x, in_w, in_b, base, drive, eta_raw, out_w, out_b)]
        if fused:
            y = native.layer_train(*leaves, positions, counts, row_mask=mask)
        else:
            mixed = native.project_mix(*leaves[:6], positions, counts, row_mask=mask)
            y = native.linear(mixed, leaves[6], leaves[7], x.dtype, row_mask=mask)
        y.backward(upstream)
        return y.detach(), [leaf.grad for leaf in leaves]

    fused_out, fused_grads = run(True)
    split_out, split_grads = run(False)
    assert torch.equal(fused_out, split_out)
    names = ("x", "in_weight", "in_bias", "base", "drive", "eta", "out_weight", "out_bias")
    for name, got, want in zip(names, fused_grads, split_grads):
        assert got is not None and torch.isfinite(got).all(), name
        assert torch.equal(got, want), name


def test_module_training_forward_takes_the_one_call_path(native, monkeypatch):
    from lsso_amd import LSSO, LSSOConfig

    calls = []
    original = native.layer_train

    def spy(*args, **kwargs):
        calls.append(1)
        return original(*args, **kwargs)

    monkeypatch.setattr(native, "layer_train", spy)
    torch.manual_seed(0)
    layer = LSSO(LSSOConfig(dim=256, num_heads=8, rank=48, bias=True)).cuda()
    x = torch.randn(2, 200, 256, device="cuda").half().requires_grad_(True)
    y = layer(x, implementation="hip")
    y.float().square().mean().backward()
    assert calls, "module training did not take the one-call layer path"
    assert x.grad is not None and torch.isfinite(x.grad).all()
