"""FP64 compact-equilibrium diagnostics (reference lsso/ball/reference.py:575-688,
lsso/ball/model.py:498-522; tests/core/test_reference.py:389-437 and
tests/core/test_model.py:123-155 in the reference)."""

from __future__ import annotations

import pytest
import torch

from lsso_amd import LSSO, LSSOConfig
from lsso_amd.ball import reference as canonical


def _problem(batch=2, heads=3, length=9, rank=4, head_dim=5, seed=70):
    generator = torch.Generator().manual_seed(seed)
    frame = canonical.qr_soft_frame(torch.randn(batch, heads, length, rank, dtype=torch.float64, generator=generator))
    raw = torch.randn(batch, heads, rank, rank, dtype=torch.float64, generator=generator)
    content = torch.randn(batch, heads, length, head_dim, dtype=torch.float64, generator=generator)
    eta = canonical.bounded_complement(torch.linspace(-0.4, 0.7, heads, dtype=torch.float64))
    compact_state = frame.mT @ content
    rhs = torch.randn(compact_state.shape, dtype=torch.float64, generator=generator)
    return frame, canonical.accretive_generator(raw), compact_state, eta, rhs


def test_token_gain_is_the_dense_operator_norm() -> None:
    frame, generator, compact_state, eta, rhs = _problem()
    out = canonical.compact_equilibrium_diagnostics(frame, generator, compact_state, eta, rhs)
    batch, heads, length, rank = frame.shape
    identity_r = torch.eye(rank, dtype=torch.float64)
    system = identity_r + generator
    reflection = 2.0 * torch.linalg.inv(system) - identity_r
    eta4 = eta.view(1, heads, 1, 1)
    dense = eta4 * torch.eye(length, dtype=torch.float64) + frame @ (reflection - eta4 * identity_r) @ frame.mT
    torch.testing.assert_close(out["q"], torch.linalg.matrix_norm(dense, ord=2), rtol=2e-11, atol=2e-12)
    torch.testing.assert_close(out["mu"], torch.linalg.eigvalsh(0.5 * (system + system.mT))[..., 0])
    state = torch.linalg.solve(system, compact_state)
    torch.testing.assert_close(out["state_ratio"], state.norm(dim=(-2, -1)) / compact_state.norm(dim=(-2, -1)))
    assert torch.all(out["q"] < 1.0)
    assert torch.all(out["mu"] > 1.0)
    assert torch.all(out["state_bound_usage"] <= 1.0 + 2e-12)
    assert torch.all(out["adjoint_bound_usage"] <= 1.0 + 2e-12)
    torch.testing.assert_close(out["contraction_slack"], 1.0 - out["q"])


def test_square_frame_has_no_complement_term() -> None:
    frame, generator, compact_state, eta, rhs = _problem(length=4, rank=4)
    out = canonical.compact_equilibrium_diagnostics(frame, generator, compact_state, eta, rhs)
    identity = torch.eye(4, dtype=torch.float64)
    reflection = 2.0 * torch.linalg.inv(identity + generator) - identity
    eta4 = eta.view(1, -1, 1, 1)
    dense = eta4 * identity + frame @ (reflection - eta4 * identity) @ frame.mT
    torch.testing.assert_close(out["q"], torch.linalg.matrix_norm(dense, ord=2), rtol=2e-11, atol=2e-12)


def test_diagnostics_reject_short_sequences_and_bad_shapes() -> None:
    frame, generator, compact_state, eta, rhs = _problem(length=3, rank=4)
    with pytest.raises(ValueError, match="N >= rank R"):
        canonical.compact_equilibrium_diagnostics(frame, generator, compact_state, eta, rhs)
    frame, generator, compact_state, eta, rhs = _problem()
    with pytest.raises(ValueError, match="adjoint_rhs must match"):
        canonical.compact_equilibrium_diagnostics(frame, generator, compact_state, eta, rhs[..., :2])
    with pytest.raises(ValueError, match="eta must have shape"):
        canonical.compact_equilibrium_diagnostics(frame, generator, compact_state, eta[:2], rhs)


def test_model_diagnostics_follow_the_masked_reference_problem() -> None:
    torch.manual_seed(71)
    layer = LSSO(LSSOConfig(dim=24, num_heads=3, rank=6, bias=True)).double().eval()
    with torch.no_grad():
        layer.core_base_raw.normal_(std=0.1)
        layer.core_drive_weight.normal_(std=0.1)
        layer.eta_raw.normal_(std=0.3)
    x = torch.randn(2, 11, 24, dtype=torch.float64)
    mask = torch.tensor([[True] * 9 + [False] * 2, [True] * 7 + [False] * 4])
    rhs = torch.randn(2, 3, 6, 8, dtype=torch.float64)
    out = layer.diagnostics(x, valid_mask=mask, adjoint_rhs=rhs)
    assert set(out) == {"q", "contraction_slack", "mu", "state_ratio", "adjoint_ratio",
                        "state_bound_usage", "adjoint_bound_usage"}
    assert all(value.shape == (2, 3) for value in out.values())
    assert all(torch.isfinite(value).all() for value in out.values())
    assert torch.all(out["q"] < 1.0)
    assert torch.all(out["state_bound_usage"] <= 1.0 + 2e-12)
    assert torch.all(out["adjoint_bound_usage"] <= 1.0 + 2e-12)


@pytest.mark.gpu
def test_native_diagnostics_certify_the_native_operator() -> None:
    """The native tape gives P^T P = I - L^-1 L^-T, I + K and Z: its
    certificates agree with the canonical torch path's on the same input."""

    from lsso_amd.ball import hip

    hip.load()
    torch.manual_seed(72)
    layer = LSSO(LSSOConfig(dim=128, num_heads=4, rank=32, bias=True)).cuda().eval()
    with torch.no_grad():
        layer.core_base_raw.normal_(std=0.1)
        layer.core_drive_weight.normal_(std=0.1)
        layer.eta_raw.normal_(std=0.3)
    x = torch.randn(2, 300, 128, generator=torch.Generator().manual_seed(73)).half().cuda()
    mask = (torch.arange(300)[None, :] < torch.tensor([[300], [120]])).cuda()
    rhs = torch.randn(2, 4, 32, 32, dtype=torch.float64, device="cuda")
    native = layer.diagnostics(x, valid_mask=mask, adjoint_rhs=rhs, implementation="hip")
    torch.cuda.synchronize()
    reference = layer.diagnostics(x.float(), valid_mask=mask, adjoint_rhs=rhs)
    for key in ("q", "mu", "state_ratio", "adjoint_ratio"):
        rel = ((native[key] - reference[key]).abs() / reference[key].abs()).max().item()
        assert rel < 2e-2, (key, rel)
    assert torch.all(native["q"] < 1.0)
    assert torch.all(native["state_bound_usage"] <= 1.0 + 1e-9)
    assert torch.all(native["adjoint_bound_usage"] <= 1.0 + 1e-9)


@pytest.mark.gpu
def test_native_diagnostics_match_the_dense_oracle_operator() -> None:
    """The native certificates against closed forms of the oracle's compact
    problem (oracle/lsso_reference.py, independent of the package's torch
    path): q = ||T||_2 of the dense N x N operator
    T = eta I + P (2 (I + K)^-1 - I - eta I) P^T, mu = lambda_min(sym(I + K)),
    and the solve / adjoint ratios from dense FP64 solves."""

    from lsso_amd.ball import hip
    from oracle import lsso_reference as oracle

    hip.load()
    torch.manual_seed(74)
    dim, heads, rank, length = 128, 4, 32, 300
    layer = LSSO(LSSOConfig(dim=dim, num_heads=heads, rank=rank, bias=True)).cuda().eval()
    with torch.no_grad():
        layer.core_base_raw.normal_(std=0.1)
        layer.core_drive_weight.normal_(std=0.1)
        layer.eta_raw.normal_(std=0.3)
    x = torch.randn(2, length, dim, generator=torch.Generator().manual_seed(75)).half()
    mask = torch.arange(length)[None, :] < torch.tensor([[length], [120]])
    rhs = torch.randn(2, heads, rank, dim // heads, dtype=torch.float64,
                      generator=torch.Generator().manual_seed(76))
    native = layer.diagnostics(x.cuda(), valid_mask=mask.cuda(), adjoint_rhs=rhs.cuda(), implementation="hip")
    torch.cuda.synchronize()

    params = {name: p.detach().float().cpu() for name, p in layer.named_parameters()}
    config = {"dim": dim, "num_heads": heads, "rank": rank, "bias": True}
    _, frame, state, _, generator, eta = oracle.compact_problem(params, config, x.float(), mask)
    frame, state, generator, eta = (t.double() for t in (frame, state, generator, eta))
    identity = torch.eye(rank, dtype=torch.float64)
    system = identity + generator
    eta4 = eta.view(1, heads, 1, 1)
    reflection = 2.0 * torch.linalg.inv(system) - identity
    dense = eta4 * torch.eye(length, dtype=torch.float64) + frame @ (reflection - eta4 * identity) @ frame.mT
    expected = {
        "q": torch.linalg.matrix_norm(dense, ord=2),
        "mu": torch.linalg.eigvalsh(0.5 * (system + system.mT))[..., 0],
        "state_ratio": torch.linalg.solve(system, state).norm(dim=(-2, -1)) / state.norm(dim=(-2, -1)),
        "adjoint_ratio": torch.linalg.solve(system.mT, rhs).norm(dim=(-2, -1)) / rhs.norm(dim=(-2, -1)),
    }
    for key, value in expected.items():
        rel = ((native[key].cpu() - value).abs() / value.abs()).max().item()
        assert rel < 2e-2, (key, rel)
