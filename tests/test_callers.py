"""The native path inside the reference's callers (GPU).

Two callers of the mixer, restated here so the test does not import them:
  - the vision adapter's token positions (reference
    integrations/timm.py:150-165): a zero-phase CLS token followed by
    centred one-dimensional patch coordinates, with optional trailing
    padding of the patch sequence;
  - the sequence runner's pre-norm residual block (reference
    experiments/train_transformers.py:480-560): LayerNorm, the mixer on the
    AMP dtype, residual, row masking, then the MLP half, trained under FP16
    autocast.
Forward outputs must stay within rel L2 5e-3 of the FP64 oracle (for the
runner, the whole block evaluated in FP64 with the oracle mixer), and
gradients within 3e-2 (reference docs/CUDA_CONTRACT.md:93-101).
"""

from __future__ import annotations

import pytest
import torch
from torch import nn

from lsso_amd import LSSO, LSSOConfig
from oracle import lsso_reference as oracle

pytestmark = pytest.mark.gpu


def _rel_l2(actual, expected) -> float:
    actual = torch.as_tensor(actual).detach().to(device="cpu", dtype=torch.float64)
    expected = torch.as_tensor(expected).detach().to(device="cpu", dtype=torch.float64)
    return float((actual - expected).norm() / expected.norm().clamp_min(1e-30))


def _vision_positions(length: int) -> torch.Tensor:
    """Zero-phase CLS, then patch coordinates centred on the patch sequence."""

    patches = torch.arange(length - 1, dtype=torch.float32) - 0.5 * (length - 2)
    return torch.cat((torch.zeros(1), patches))


@pytest.mark.parametrize("padded", (False, True))
def test_vision_token_positions_match_fp64_oracle(native, padded: bool) -> None:
    torch.manual_seed(197)
    config = LSSOConfig(dim=192, num_heads=3, rank=16, bias=True)
    layer = LSSO(config).cuda().eval()
    with torch.no_grad():
        layer.core_base_raw.normal_(std=0.05)
        layer.core_drive_weight.normal_(std=0.05)
    length = 197                      # CLS + 14 x 14 patches
    positions = _vision_positions(length)
    x = torch.randn(2, length, config.dim, generator=torch.Generator().manual_seed(5)).half()
    mask = None
    if padded:
        mask = torch.ones(2, length, dtype=torch.bool)
        mask[1, 150:] = False         # a smaller image: trailing patch padding
        x[~mask] = float("nan")
    with torch.no_grad():
        out = layer(x.cuda(), valid_mask=None if mask is None else mask.cuda(),
                    position_ids=positions.cuda(), implementation="hip")
    params = {name: p.detach().double().cpu() for name, p in layer.named_parameters()}
    expected = oracle.lsso_forward(params, {"dim": 192, "num_heads": 3, "rank": 16, "bias": True},
                                   x.double(), mask, positions)
    assert torch.isfinite(out).all()
    if mask is not None:
        assert torch.count_nonzero(out.cpu()[~mask]) == 0
    assert _rel_l2(out, expected) <= 5e-3


class _PreNormBlock(nn.Module):
    """LayerNorm -> LSSO (AMP dtype) -> residual -> mask -> MLP -> mask."""

    def __init__(self, dim: int, heads: int, rank: int, implementation: str) -> None:
        super().__init__()
        self.implementation = implementation
        self.norm1 = nn.LayerNorm(dim)
        self.mixer = LSSO(LSSOConfig(dim=dim, num_heads=heads, rank=rank, bias=True))
        self.norm2 = nn.LayerNorm(dim)
        self.mlp = nn.Sequential(nn.Linear(dim, 2 * dim), nn.GELU(), nn.Linear(2 * dim, dim))

    def forward(self, x: torch.Tensor, valid_mask: torch.Tensor) -> torch.Tensor:
        normalized = self.norm1(x)
        if torch.is_autocast_enabled():
            normalized = normalized.to(dtype=torch.get_autocast_dtype("cuda"))
        mixed = self.mixer(normalized, valid_mask=valid_mask, implementation=self.implementation)
        x = x + mixed
        x = torch.where(valid_mask[:, :, None], x, torch.zeros_like(x))
        x = x + self.mlp(self.norm2(x))
        return torch.where(valid_mask[:, :, None], x, torch.zeros_like(x))


def _oracle_block(block: _PreNormBlock, x: torch.Tensor, valid_mask: torch.Tensor):
    """The same block in FP64 on the CPU with the mixer replaced by the oracle
    (oracle.lsso_forward): output, input gradient and parameter gradients of
    mean(y^2)."""

    params = {name: p.detach().double().cpu().requires_grad_(True) for name, p in block.named_parameters()}
    mixer = {name[len("mixer."):]: value for name, value in params.items() if name.startswith("mixer.")}
    dim = block.norm1.normalized_shape[0]
    config = {"dim": dim, "num_heads": block.mixer.config.num_heads, "rank": block.mixer.config.rank,
              "bias": True}
    leaf = x.detach().double().cpu().requires_grad_(True)
    mask = valid_mask.cpu()
    keep = mask[:, :, None]
    normalized = nn.functional.layer_norm(leaf, (dim,), params["norm1.weight"], params["norm1.bias"],
                                          block.norm1.eps)
    hidden = leaf + oracle.lsso_forward(mixer, config, normalized, mask)
    hidden = torch.where(keep, hidden, torch.zeros_like(hidden))
    inner = nn.functional.layer_norm(hidden, (dim,), params["norm2.weight"], params["norm2.bias"],
                                     block.norm2.eps)
    inner = nn.functional.linear(inner, params["mlp.0.weight"], params["mlp.0.bias"])
    inner = nn.functional.linear(nn.functional.gelu(inner), params["mlp.2.weight"], params["mlp.2.bias"])
    y = torch.where(keep, hidden + inner, torch.zeros_like(hidden))
    y.square().mean().backward()
    return y.detach(), leaf.grad, {name: value.grad for name, value in params.items()}


def test_pre_norm_residual_block_trains_like_the_fp64_oracle(native) -> None:
    """The block under FP16 autocast on the native path against the same
    block in FP64 with the oracle mixer; the block with
    implementation="reference" (the package's torch path) is run beside it
    and must agree with the oracle to the same bar."""

    torch.manual_seed(480)
    dim, heads, rank, batch, length = 128, 4, 32, 3, 300
    native_block = _PreNormBlock(dim, heads, rank, "hip").cuda()
    with torch.no_grad():
        native_block.mixer.core_base_raw.normal_(std=0.05)
        native_block.mixer.core_drive_weight.normal_(std=0.05)
    reference_block = _PreNormBlock(dim, heads, rank, "reference").cuda()
    reference_block.load_state_dict(native_block.state_dict())
    x = torch.randn(batch, length, dim, device="cuda", generator=torch.Generator(device="cuda").manual_seed(2))
    mask = torch.arange(length, device="cuda")[None, :] < torch.tensor([[300], [211], [64]], device="cuda")

    def run(block):
        leaf = x.clone().requires_grad_(True)
        with torch.autocast(device_type="cuda", dtype=torch.float16):
            y = block(leaf, mask)
        y.float().square().mean().backward()
        return y.detach(), leaf.grad, {name: p.grad for name, p in block.named_parameters()}

    y_oracle, gx_oracle, g_oracle = _oracle_block(native_block, x, mask)
    for block in (native_block, reference_block):
        y, gx, grads = run(block)
        assert torch.isfinite(y).all()
        assert _rel_l2(y, y_oracle) <= 5e-3, block.implementation
        assert _rel_l2(gx, gx_oracle) <= 3e-2, block.implementation
        for name, grad in grads.items():
            assert grad is not None and torch.isfinite(grad).all(), name
            assert _rel_l2(grad, g_oracle[name]) <= 3e-2, (block.implementation, name,
                                                           _rel_l2(grad, g_oracle[name]))
