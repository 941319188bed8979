"""Pin the CPU oracle before trusting it (CPU only).

1. Golden vectors written by the real reference (tests/golden/make_golden.py)
   pin the FP32 operation order, BF16/FP16 rounding boundaries, the default
   init under a seed and the FP64 outputs.
2. Closed forms pin the mathematics independently of the reference code.
3. Planted mistakes in the oracle must be caught by those checks.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import gram_cholesky
from oracle import lsso_reference as oracle

GOLDEN = Path(__file__).resolve().parent / "golden"


def _load(name: str) -> dict[str, np.ndarray]:
    with np.load(GOLDEN / name, allow_pickle=False) as data:
        return {key: data[key] for key in data.files}


def _params(data: dict[str, np.ndarray]) -> dict[str, torch.Tensor]:
    return {
        key.split(":", 1)[1]: torch.from_numpy(value)
        for key, value in data.items()
        if key.startswith("param:")
    }


def _rel_l2(actual, expected) -> float:
    actual = torch.as_tensor(actual, dtype=torch.float64)
    expected = torch.as_tensor(expected, dtype=torch.float64)
    return float((actual - expected).norm() / expected.norm().clamp_min(1e-300))


C1 = {"dim": 192, "num_heads": 3, "rank": 16, "bias": False}


def test_oracle_init_reproduces_reference_default_state() -> None:
    data = _load("c1_default.npz")
    params = oracle.init_params(C1, seed=0)
    for name, value in _params(data).items():
        assert torch.equal(params[name], value), name


def test_oracle_fp32_forward_matches_reference_cpu_path() -> None:
    data = _load("c1_default.npz")
    params = _params(data)
    x = torch.from_numpy(data["x"])
    y = oracle.lsso_forward(params, C1, x)
    assert y.dtype == torch.float32
    # Same op order as the reference; only BLAS blocking can move an FP32 ulp.
    assert _rel_l2(y, data["y32"]) < 2e-6
    projected, frame, compact_state, _content, generator, eta = oracle.compact_problem(params, C1, x)
    assert torch.equal(projected.float(), torch.from_numpy(data["projected"]))
    assert _rel_l2(frame, data["frame"]) < 1e-5
    assert _rel_l2(compact_state, data["compact_state"]) < 1e-5
    assert _rel_l2(generator, data["generator"]) < 1e-6
    assert torch.equal(eta, torch.from_numpy(data["eta"]))


def test_oracle_fp64_forward_matches_reference() -> None:
    data = _load("c1_default.npz")
    params = {k: v.double() for k, v in _params(data).items()}
    y = oracle.lsso_forward(params, C1, torch.from_numpy(data["x"]).double())
    assert _rel_l2(y, data["y64"]) < 1e-12


@pytest.mark.parametrize("precision", ("32", "64"))
def test_oracle_masked_per_sample_positions_match_reference(precision: str) -> None:
    data = _load("masked.npz")
    config = {"dim": 24, "num_heads": 2, "rank": 8, "bias": True}
    params = _params(data)
    x = torch.from_numpy(data["x"])
    if precision == "64":
        params = {k: v.double() for k, v in params.items()}
        x = x.double()
    mask = torch.from_numpy(data["mask"])
    positions = torch.from_numpy(data["position_ids"])
    y = oracle.lsso_forward(params, config, x, mask, positions)
    expected = data[f"y{precision}"]
    assert torch.isfinite(y).all()
    assert torch.count_nonzero(y[~mask]) == 0
    assert _rel_l2(y, expected) < (1e-12 if precision == "64" else 2e-6)


@pytest.mark.parametrize("precision", ("32", "64"))
def test_oracle_rank48_gradients_match_reference(precision: str) -> None:
    data = _load("rank48_backward.npz")
    config = {"dim": 96, "num_heads": 2, "rank": 48, "bias": True}
    dtype = torch.float64 if precision == "64" else torch.float32
    params = {k: v.to(dtype).requires_grad_() for k, v in _params(data).items()}
    x = torch.from_numpy(data["x"]).to(dtype).requires_grad_()
    y = oracle.lsso_forward(params, config, x)
    y.square().mean().backward()
    limit = 1e-11 if precision == "64" else 1e-5
    assert _rel_l2(y.detach(), data[f"y{precision}"]) < limit
    assert _rel_l2(x.grad, data[f"grad{precision}:x"]) < limit
    for name, value in params.items():
        assert _rel_l2(value.grad, data[f"grad{precision}:{name}"]) < limit, name


@pytest.mark.parametrize("tag", ("r32", "r48"))
def test_oracle_abi_fast_mix_matches_reference(tag: str) -> None:
    data = _load("fast_mix.npz")
    mixed = oracle.fast_mix_fp64(
        torch.from_numpy(data[f"{tag}:projected"]),
        torch.from_numpy(data[f"{tag}:base"]),
        torch.from_numpy(data[f"{tag}:drive"]),
        torch.from_numpy(data[f"{tag}:eta_raw"]),
    )
    assert _rel_l2(mixed, data[f"{tag}:mixed64"]) < 1e-12


# -- closed forms ------------------------------------------------------------
def test_frame_identity_and_contraction() -> None:
    torch.manual_seed(0)
    relation = torch.randn(3, 2, 19, 8, dtype=torch.float64)
    frame = oracle.qr_soft_frame(relation)
    eye = torch.eye(8, dtype=torch.float64)
    expected = relation @ torch.linalg.solve(eye + relation.mT @ relation, relation.mT)
    torch.testing.assert_close(frame @ frame.mT, expected, rtol=1e-12, atol=1e-12)
    assert torch.all(torch.linalg.matrix_norm(frame, ord=2) <= 1.0 + 1e-12)


def test_gram_cholesky_restatement_agrees_with_qr_oracle() -> None:
    generator = torch.Generator().manual_seed(3)
    projected = torch.randn(2, 37, 2 * (32 + 24), generator=generator, dtype=torch.float64)
    base = 0.1 * torch.randn(2, 32, 32, generator=generator, dtype=torch.float64)
    drive = 0.1 * torch.randn(2, 24, 32, generator=generator, dtype=torch.float64)
    eta_raw = torch.tensor([0.3, -0.8], dtype=torch.float64)
    positions = torch.randn(2, 37, generator=generator, dtype=torch.float64) * 50
    counts = torch.tensor([37.0, 20.0], dtype=torch.float64)
    qr = oracle.fast_mix_fp64(projected, base, drive, eta_raw, positions, counts)
    chol = gram_cholesky.mix(projected.numpy(), base.numpy(), drive.numpy(), eta_raw.numpy(),
                             positions.numpy(), counts.numpy())
    assert _rel_l2(qr, chol) < 1e-11


def test_dense_operator_brute_force_on_tiny_input() -> None:
    generator = torch.Generator().manual_seed(4)
    projected = torch.randn(1, 6, 2 * (16 + 3), generator=generator, dtype=torch.float64)
    base = 0.2 * torch.randn(2, 16, 16, generator=generator, dtype=torch.float64)
    drive = 0.2 * torch.randn(2, 3, 16, generator=generator, dtype=torch.float64)
    eta_raw = torch.tensor([0.4, -0.2], dtype=torch.float64)
    mixed = oracle.fast_mix_fp64(projected, base, drive, eta_raw).numpy()
    for h in range(2):
        operator, content = gram_cholesky.dense_operator(projected.numpy(), base.numpy(), drive.numpy(),
                                                         eta_raw.numpy(), 0, h)
        np.testing.assert_allclose(mixed[0, :, 3 * h:3 * h + 3], operator @ content, rtol=1e-11, atol=1e-12)


def test_default_init_point_is_the_complement_projection() -> None:
    """Theta0 = W_drive = 0 gives K = I, U = Z/2, Y = eta (C - P P^T C)."""

    generator = torch.Generator().manual_seed(5)
    heads, rank, head_dim, length = 2, 16, 5, 23
    projected = torch.randn(1, length, heads * (rank + head_dim), generator=generator, dtype=torch.float64)
    base = torch.zeros(heads, rank, rank, dtype=torch.float64)
    drive = torch.zeros(heads, head_dim, rank, dtype=torch.float64)
    eta_raw = torch.tensor([0.6, -1.1], dtype=torch.float64)
    mixed = oracle.fast_mix_fp64(projected, base, drive, eta_raw)
    eta = (1 - torch.finfo(torch.float64).eps) * torch.tanh(eta_raw)
    positions = torch.arange(length, dtype=torch.float64) - 0.5 * (length - 1)
    relation = projected[..., : heads * rank].view(1, length, heads, rank).transpose(1, 2)
    content = projected[..., heads * rank:].view(1, length, heads, head_dim).transpose(1, 2)
    a = oracle.rank_rotary(relation, positions.view(1, -1)) / length ** 0.5
    eye = torch.eye(rank, dtype=torch.float64)
    ppt = a @ torch.linalg.solve(eye + a.mT @ a, a.mT)
    expected = eta.view(1, heads, 1, 1) * (content - ppt @ content)
    torch.testing.assert_close(mixed, expected.transpose(1, 2).reshape(1, length, -1), rtol=1e-11, atol=1e-12)


def test_rotation_preserves_norms_and_composes() -> None:
    generator = torch.Generator().manual_seed(6)
    relation = torch.randn(2, 1, 7, 16, generator=generator, dtype=torch.float64)
    p = torch.randn(2, 7, generator=generator, dtype=torch.float64) * 30
    q = torch.randn(2, 7, generator=generator, dtype=torch.float64) * 30
    rotated = oracle.rank_rotary(relation, p)
    torch.testing.assert_close(rotated.norm(dim=-1), relation.norm(dim=-1), rtol=1e-13, atol=1e-13)
    torch.testing.assert_close(
        oracle.rank_rotary(oracle.rank_rotary(relation, p), q), oracle.rank_rotary(relation, p + q),
        rtol=1e-11, atol=1e-11,
    )


# -- planted mistakes --------------------------------------------------------
def test_planted_mistakes_in_the_oracle_are_caught(monkeypatch: pytest.MonkeyPatch) -> None:
    data = _load("c1_default.npz")
    params = {k: v.double() for k, v in _params(data).items()}
    x = torch.from_numpy(data["x"]).double()
    baseline = oracle.lsso_forward(params, C1, x)
    assert _rel_l2(baseline, data["y64"]) < 1e-12

    original_rotary = oracle.rank_rotary

    def wrong_sign_rotary(relation, positions):
        return original_rotary(relation, -positions)

    monkeypatch.setattr(oracle, "rank_rotary", wrong_sign_rotary)
    assert _rel_l2(oracle.lsso_forward(params, C1, x), data["y64"]) > 1e-4
    monkeypatch.undo()

    original_frame = oracle.qr_soft_frame

    def unscaled_frame(relation):
        return original_frame(relation * 2.0)

    monkeypatch.setattr(oracle, "qr_soft_frame", unscaled_frame)
    assert _rel_l2(oracle.lsso_forward(params, C1, x), data["y64"]) > 1e-4
    monkeypatch.undo()

    # A transposed factor Gram (F^T F instead of F F^T) must break the
    # masked fixture, whose compact core is non-zero.
    masked = _load("masked.npz")
    config = {"dim": 24, "num_heads": 2, "rank": 8, "bias": True}
    mparams = {k: v.double() for k, v in _params(masked).items()}
    mx = torch.from_numpy(masked["x"]).double()
    mask = torch.from_numpy(masked["mask"])
    positions = torch.from_numpy(masked["position_ids"])
    original_generator = oracle.accretive_generator

    def transposed_generator(raw):
        k = original_generator(raw)
        diagonal = torch.diagonal(raw, dim1=-2, dim2=-1)
        factor = torch.tril(raw, -1) + torch.diag_embed(
            torch.nn.functional.softplus(diagonal + oracle.SOFTPLUS_ONE_OFFSET)
        )
        return k - factor @ factor.mT + factor.mT @ factor

    monkeypatch.setattr(oracle, "accretive_generator", transposed_generator)
    broken = oracle.lsso_forward(mparams, config, mx, mask, positions)
    assert _rel_l2(broken, masked["y64"]) > 1e-4
