"""Public API, configuration, checkpoint contract and the PyTorch reference
path (CPU).  Mirrors the reference's core contract tests
(tests/core/test_model.py, tests/core/test_public_api.py)."""

from __future__ import annotations

import copy
from pathlib import Path

import numpy as np
import pytest
import torch

import lsso_amd
from lsso_amd import CoreMode, LSSO, LSSOConfig
from lsso_amd.ball import reference as canonical
from oracle import lsso_reference as oracle

GOLDEN = Path(__file__).resolve().parent / "golden"


def _rel_l2(actual, expected) -> float:
    actual = torch.as_tensor(actual).detach().to(torch.float64)
    expected = torch.as_tensor(expected).detach().to(torch.float64)
    return float((actual - expected).norm() / expected.norm().clamp_min(1e-300))


def _params(layer: LSSO, dtype=torch.float64) -> dict[str, torch.Tensor]:
    return {name: p.detach().to(dtype) for name, p in layer.named_parameters()}


def _config(layer: LSSO) -> dict:
    c = layer.config
    return {"dim": c.dim, "num_heads": c.num_heads, "rank": c.rank, "bias": c.bias,
            "core_mode": c.core_mode.value, "rank_rotary": c.rank_rotary}


def test_public_api_is_narrow() -> None:
    assert set(lsso_amd.__all__) == {"CoreMode", "LSSO", "LSSOConfig", "__version__"}
    assert lsso_amd.__version__ == "0.6.3"


def test_default_is_the_complete_dynamic_variant() -> None:
    config = LSSOConfig(dim=24, num_heads=3, rank=6)
    assert config.core_mode is CoreMode.DYNAMIC
    assert config.rank_rotary and not config.bias
    assert config.head_dim == 8


@pytest.mark.parametrize(("keyword", "value"), [("dim", 8.0), ("num_heads", True), ("rank", 4.0)])
def test_configuration_requires_integer_dimensions(keyword, value) -> None:
    arguments = {"dim": 8, "num_heads": 2, "rank": 4}
    arguments[keyword] = value
    with pytest.raises(TypeError, match=keyword):
        LSSOConfig(**arguments)


def test_configuration_validation() -> None:
    with pytest.raises(TypeError, match="rank_rotary"):
        LSSOConfig(8, 2, rank=4, rank_rotary="false")
    with pytest.raises(TypeError, match="bias"):
        LSSOConfig(8, 2, rank=4, bias=1)
    with pytest.raises(ValueError, match="divisible"):
        LSSOConfig(10, 3, rank=4)
    with pytest.raises(ValueError, match="even rank"):
        LSSOConfig(8, 2, rank=5)
    with pytest.raises(ValueError, match="core_mode"):
        LSSOConfig(8, 2, rank=4, core_mode="unknown")
    assert LSSOConfig(8, 2, rank=4, core_mode="zero").core_mode is CoreMode.ZERO
    with pytest.raises(TypeError):
        LSSOConfig(8, 2, eta=0.9)


@pytest.mark.parametrize(
    ("mode", "present", "absent"),
    [
        (CoreMode.DYNAMIC, {"core_base_raw", "core_drive_weight"}, set()),
        (CoreMode.STATIC, {"core_base_raw"}, {"core_drive_weight"}),
        (CoreMode.ZERO, set(), {"core_base_raw", "core_drive_weight"}),
    ],
)
def test_core_modes_create_only_owned_parameters(mode, present, absent) -> None:
    names = set(dict(LSSO(LSSOConfig(16, 2, rank=4, core_mode=mode)).named_parameters()))
    assert {"eta_raw", "w_bc.weight", "w_o.weight"} <= names
    assert present <= names
    assert names.isdisjoint(absent)


def test_learned_complement_starts_at_0_9() -> None:
    layer = LSSO(LSSOConfig(dim=8, num_heads=2, rank=4))
    torch.testing.assert_close(layer.complement(), torch.full((2,), 0.9))


def test_reference_checkpoint_loads_unchanged() -> None:
    """A state_dict holding the reference's parameters and contract v12
    loads into lsso_amd.LSSO (reference lsso/ball/model.py:79-140)."""

    with np.load(GOLDEN / "c1_default.npz") as data:
        state = {k.split(":", 1)[1]: torch.from_numpy(data[k]) for k in data.files if k.startswith("param:")}
    layer = LSSO(LSSOConfig(dim=192, num_heads=3, rank=16))
    state["_extra_state"] = layer.get_extra_state()
    layer.load_state_dict(state, strict=True)
    for name, parameter in layer.named_parameters():
        assert torch.equal(parameter.detach(), state[name])


def test_default_init_matches_the_reference_under_a_seed() -> None:
    with np.load(GOLDEN / "c1_default.npz") as data:
        expected = {k.split(":", 1)[1]: data[k] for k in data.files if k.startswith("param:")}
    torch.manual_seed(0)
    layer = LSSO(LSSOConfig(dim=192, num_heads=3, rank=16))
    for name, parameter in layer.named_parameters():
        np.testing.assert_array_equal(parameter.detach().numpy(), expected[name])


def test_checkpoint_contract_round_trips_and_rejects_mismatch() -> None:
    source = LSSO(LSSOConfig(16, 2, rank=4, rank_rotary=True))
    target = LSSO(LSSOConfig(16, 2, rank=4))
    target.load_state_dict(source.state_dict(), strict=True)
    other = LSSO(LSSOConfig(16, 2, rank=4, rank_rotary=False))
    for strict in (True, False):
        with pytest.raises(RuntimeError, match="checkpoint contract"):
            other.load_state_dict(source.state_dict(), strict=strict)
    state = copy.deepcopy(source.state_dict())
    assert state["_extra_state"]["version"] == 12
    assert state["_extra_state"]["numerics"] == "tf32-wbc-ieee-fgram-tc16-v6"
    del state["_extra_state"]
    for strict in (True, False):
        with pytest.raises(RuntimeError, match="missing its configuration contract"):
            target.load_state_dict(state, strict=strict)


def test_checkpoint_contract_cannot_be_bypassed_in_a_parent_load() -> None:
    class Container(torch.nn.Module):
        def __init__(self) -> None:
            super().__init__()
            self.mixer = LSSO(LSSOConfig(16, 2, rank=4))

    state = copy.deepcopy(Container().state_dict())
    del state["mixer._extra_state"]
    with pytest.raises(RuntimeError, match="missing its configuration contract"):
        Container().load_state_dict(state, strict=False)


# -- reference path ------------------------------------------------------------
@pytest.mark.parametrize("core_mode", list(CoreMode))
@pytest.mark.parametrize("rank_rotary", (False, True))
def test_reference_path_matches_oracle_in_fp64(core_mode, rank_rotary) -> None:
    torch.manual_seed(10)
    layer = LSSO(LSSOConfig(dim=24, num_heads=3, rank=6, core_mode=core_mode,
                            rank_rotary=rank_rotary, bias=True)).double()
    with torch.no_grad():
        for parameter in (layer.core_base_raw, layer.core_drive_weight):
            if parameter is not None:
                parameter.normal_(std=0.15)
    x = torch.randn(2, 11, 24, dtype=torch.float64)
    expected = oracle.lsso_forward(_params(layer), _config(layer), x)
    torch.testing.assert_close(layer(x), expected, rtol=1e-10, atol=1e-11)


def test_reference_path_fp32_matches_reference_golden() -> None:
    with np.load(GOLDEN / "c1_default.npz") as data:
        x = torch.from_numpy(data["x"])
        y32 = data["y32"]
        state = {k.split(":", 1)[1]: torch.from_numpy(data[k]) for k in data.files if k.startswith("param:")}
    layer = LSSO(LSSOConfig(dim=192, num_heads=3, rank=16))
    with torch.no_grad():
        for name, parameter in layer.named_parameters():
            parameter.copy_(state[name])
        y = layer(x)
    # The Gram-Cholesky frame differs from the reference's QR frame only by
    # FP32 rounding, amplified at most by a BF16 rounding step of the mix.
    assert _rel_l2(y, y32) < 1e-3


def test_reference_path_masked_golden() -> None:
    with np.load(GOLDEN / "masked.npz") as data:
        x = torch.from_numpy(data["x"])
        mask = torch.from_numpy(data["mask"])
        positions = torch.from_numpy(data["position_ids"])
        y64 = data["y64"]
        state = {k.split(":", 1)[1]: torch.from_numpy(data[k]) for k in data.files if k.startswith("param:")}
    layer = LSSO(LSSOConfig(dim=24, num_heads=2, rank=8, bias=True)).double()
    with torch.no_grad():
        for name, parameter in layer.named_parameters():
            parameter.copy_(state[name])
        y = layer(x.double(), valid_mask=mask, position_ids=positions)
    assert _rel_l2(y, y64) < 1e-10
    assert torch.count_nonzero(y[~mask]) == 0


def test_gapped_nan_padding_matches_cropped_sequence() -> None:
    torch.manual_seed(17)
    layer = LSSO(LSSOConfig(dim=16, num_heads=2, rank=8, bias=True)).double().eval()
    clean = torch.randn(1, 8, 16, dtype=torch.float64)
    mask = torch.tensor([[True, False, True, False, False, True, False, False]])
    positions = (3 * torch.arange(8) + 11).view(1, 8)
    poisoned = torch.where(mask[:, :, None], clean, torch.full_like(clean, float("nan")))
    output = layer(poisoned, valid_mask=mask, position_ids=positions)
    kept = mask[0].nonzero(as_tuple=False).flatten()
    expected = layer(clean[:, kept], position_ids=positions[:, kept])
    torch.testing.assert_close(output[:, kept], expected, rtol=2e-11, atol=2e-11)
    assert torch.count_nonzero(output[:, ~mask[0]]) == 0


def test_all_masked_returns_zero() -> None:
    layer = LSSO(LSSOConfig(16, 2, rank=8, bias=True)).double()
    x = torch.full((2, 5, 16), float("nan"), dtype=torch.float64)
    assert torch.count_nonzero(layer(x, valid_mask=torch.zeros(2, 5, dtype=torch.bool))) == 0


def test_positions_are_shift_invariant_and_centered_before_casting() -> None:
    torch.manual_seed(18)
    layer = LSSO(LSSOConfig(dim=16, num_heads=2, rank=6)).double()
    x = torch.randn(2, 9, 16, dtype=torch.float64)
    positions = torch.arange(9).view(1, 9).expand(2, 9)
    torch.testing.assert_close(layer(x, position_ids=positions + 100_000_000),
                               layer(x, position_ids=positions), rtol=2e-11, atol=2e-11)
    layer32 = LSSO(LSSOConfig(dim=16, num_heads=2, rank=6)).eval()
    x32 = torch.randn(2, 9, 16)
    torch.testing.assert_close(layer32(x32, position_ids=torch.arange(9, dtype=torch.float64) + 1e12),
                               layer32(x32, position_ids=torch.arange(9, dtype=torch.float64)),
                               rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(layer32(x32, position_ids=torch.arange(9) + 2 ** 40),
                               layer32(x32, position_ids=torch.arange(9)), rtol=1e-5, atol=1e-6)


def test_input_validation() -> None:
    layer = LSSO(LSSOConfig(8, 2, rank=4))
    with pytest.raises(ValueError, match="sequence length"):
        layer(torch.empty(2, 0, 8))
    with pytest.raises(TypeError, match="torch.bool"):
        layer(torch.randn(1, 3, 8), valid_mask=torch.tensor([[1, 0, 1]]))
    with pytest.raises(ValueError, match="'reference', 'hip' or 'cuda'"):
        layer(torch.randn(1, 3, 8), implementation="automatic")
    for implementation in ("reference", "hip", "cuda"):
        with pytest.raises(ValueError, match="batch size"):
            layer(torch.empty(0, 3, 8), implementation=implementation)
    with pytest.raises(TypeError, match="floating-point"):
        layer(torch.randn(1, 3, 8).to(torch.int32))


def test_dynamic_zero_init_receives_gradient_on_the_reference_path() -> None:
    torch.manual_seed(14)
    layer = LSSO(LSSOConfig(16, 2, rank=4)).double()
    layer(torch.randn(3, 9, 16, dtype=torch.float64)).square().mean().backward()
    assert torch.count_nonzero(layer.core_base_raw.grad) > 0
    assert torch.count_nonzero(layer.core_drive_weight.grad) > 0


@pytest.mark.parametrize(
    "config",
    [
        LSSOConfig(32, 2, rank=16, core_mode=CoreMode.STATIC),
        LSSOConfig(32, 2, rank=16, rank_rotary=False),
        LSSOConfig(32, 2, rank=24),
    ],
)
@pytest.mark.parametrize("implementation", ("hip", "cuda"))
def test_native_dispatch_rejects_unsupported_contracts(config, implementation) -> None:
    layer = LSSO(config)
    with pytest.raises(ValueError, match=f"implementation='{implementation}'"):
        layer(torch.randn(1, 4, config.dim), implementation=implementation)


@pytest.mark.parametrize(("rank", "head_dim"), [(16, 1), (32, 17), (48, 256), (64, 384)])
def test_native_dispatch_accepts_supported_ranks_and_any_head_dim(rank, head_dim) -> None:
    layer = LSSO(LSSOConfig(dim=2 * head_dim, num_heads=2, rank=rank))
    x = torch.randn(1, 4, 2 * head_dim).half()
    with pytest.raises(ValueError, match="CUDA tensor"):
        layer(x, implementation="hip")


def test_native_dispatch_rejects_position_gradients() -> None:
    layer = LSSO(LSSOConfig(dim=32, num_heads=2, rank=16))
    positions = torch.arange(5, dtype=torch.float32, requires_grad=True)
    with pytest.raises(ValueError, match="does not support gradients"):
        layer(torch.randn(1, 5, 32), position_ids=positions, implementation="hip")


def test_canonical_frame_equals_the_qr_frame() -> None:
    torch.manual_seed(1)
    relation = torch.randn(2, 3, 21, 8, dtype=torch.float64)
    torch.testing.assert_close(canonical.qr_soft_frame(relation), oracle.qr_soft_frame(relation),
                               rtol=1e-11, atol=1e-12)
