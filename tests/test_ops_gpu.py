"""``torch.ops.lsso_equilibrium`` on the device (GPU).

The registered operators run the library's kernels: their results are
bitwise those of the ctypes entry points they wrap, the training forward's
output equals the inference output, the backward's gradients equal
``hip.backward``'s, and a compiled function calling them traces as one graph
(reference call sites lsso/ball/cuda.py:231, 269, 305).  ``fast_mix`` now
reaches the library through these operators; its gradients are checked
against FP64 autograd of the oracle.
"""

from __future__ import annotations

import pytest
import torch

from oracle import lsso_reference as oracle

pytestmark = pytest.mark.gpu


def _inputs(batch=2, length=97, heads=3, rank=32, head_dim=24, seed=5, scale=0.1):
    generator = torch.Generator().manual_seed(seed)
    projected = torch.randn(batch, length, heads * (rank + head_dim), generator=generator).bfloat16()
    base = scale * torch.randn(heads, rank, rank, generator=generator)
    drive = scale * torch.randn(heads, head_dim, rank, generator=generator)
    eta = scale * torch.randn(heads, generator=generator)
    positions = torch.arange(length, dtype=torch.float32)
    positions = positions - positions.mean()
    return [t.cuda() for t in (projected, base, drive, eta, positions)]


@pytest.mark.parametrize("rank", (16, 32, 48, 64))
def test_operators_are_the_library_entry_points(native, rank) -> None:
    projected, base, drive, eta, positions = _inputs(rank=rank)
    ops = torch.ops.lsso_equilibrium
    assert ops.contract_version() == native._NATIVE_CONTRACT_VERSION
    with torch.no_grad():
        expected = native.forward_inference(projected, base, drive, eta, positions)
        output = ops.forward_inference(projected, base, drive, eta, positions)
        train_output, tape, pivots = ops.forward_train(projected, base, drive, eta, positions)
        _out, expected_tape = native.forward_train(projected, base, drive, eta, positions)
    assert torch.equal(output, expected)
    assert torch.equal(train_output, expected)
    assert torch.equal(tape, expected_tape)
    assert pivots.numel() == 0 and pivots.dtype == torch.int32 and pivots.is_cuda
    grad_output = torch.randn(output.shape, generator=torch.Generator().manual_seed(7)).bfloat16().cuda()
    grads = ops.backward(grad_output, projected, base, drive, eta, tape, pivots, positions)
    expected_grads = native.backward(grad_output, projected, base, drive, eta, tape, positions)
    for actual, wanted in zip(grads, expected_grads):
        assert torch.equal(actual, wanted)


def test_forward_operators_reject_autograd_on_the_device(native) -> None:
    projected, base, drive, eta, _positions = _inputs()
    base.requires_grad_(True)
    with pytest.raises(RuntimeError, match="inference-only entry point"):
        torch.ops.lsso_equilibrium.forward_inference(projected, base, drive, eta)
    with pytest.raises(RuntimeError, match="private tape-producing entry point"):
        torch.ops.lsso_equilibrium.forward_train(projected, base, drive, eta)


def test_fast_mix_gradients_through_the_operators(native) -> None:
    projected, base, drive, eta, positions = _inputs(rank=48, head_dim=32, length=65)
    leaves = [t.detach().clone().requires_grad_(True) for t in (projected, base, drive, eta)]
    output = native.fast_mix(*leaves, positions)
    weight = torch.randn(output.shape, generator=torch.Generator().manual_seed(11)).cuda()
    (output.float() * weight).sum().backward()
    cpu = [t.detach().cpu().double().requires_grad_(True) for t in (projected, base, drive, eta)]
    expected = oracle.fast_mix_fp64(*cpu, positions.cpu())
    (expected * weight.cpu().double()).sum().backward()
    for leaf, reference in zip(leaves, cpu):
        error = (leaf.grad.double().cpu() - reference.grad).norm() / reference.grad.norm()
        assert torch.isfinite(leaf.grad).all()
        assert float(error) <= 3e-2


def test_compiled_caller_traces_the_operators_as_one_graph(native) -> None:
    projected, base, drive, eta, positions = _inputs(rank=16, head_dim=16, length=40)

    def mixer(projected, base, drive, eta, positions):
        return torch.ops.lsso_equilibrium.forward_inference(projected, base, drive, eta, positions).float() * 2.0

    compiled = torch.compile(mixer, backend="aot_eager", fullgraph=True)
    with torch.no_grad():
        expected = mixer(projected, base, drive, eta, positions)
        assert torch.equal(compiled(projected, base, drive, eta, positions), expected)
