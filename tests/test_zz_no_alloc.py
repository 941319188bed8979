"""lsso_hip_mixer_forward_static, the allocation-free mixer forward, called
through the C ABI: its output (and tape) must equal lsso_hip_mixer_forward's
bit for bit, call after call on the one static scratch, including a second
call with a smaller geometry that reuses the array the first one filled."""

from __future__ import annotations

import ctypes

import pytest
import torch

from lsso_amd.ball import hip

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def library():
    if not torch.cuda.is_available():
        pytest.skip("needs an MI355X")
    hip.load()
    return hip._library()


def _inputs(batch, length, heads, rank, head_dim, seed, masked=False):
    generator = torch.Generator().manual_seed(seed)
    projected = torch.randn(batch, length, heads * (rank + head_dim), generator=generator)
    base = 0.05 * torch.randn(heads, rank, rank, generator=generator)
    drive = 0.05 * torch.randn(heads, head_dim, rank, generator=generator)
    eta_raw = 0.5 * torch.randn(heads, generator=generator)
    positions = counts = None
    if masked:
        counts = torch.randint(length // 4, length + 1, (batch,), generator=generator)
        keep = torch.arange(length)[None, :] < counts[:, None]
        projected = projected * keep[..., None]
        positions = torch.randn(batch, length, generator=generator).cumsum(1)
        positions = torch.where(keep, positions - positions.mean(1, keepdim=True), 0.0)
        counts = counts.float()
    device = torch.device("cuda", 0)
    return (projected.bfloat16().to(device), base.to(device), drive.to(device),
            eta_raw.to(device), None if positions is None else positions.to(device),
            None if counts is None else counts.to(device))


def _shape_of(projected, base, drive):
    batch, length, _ = projected.shape
    return hip.MixerShape(batch, length, base.shape[0], base.shape[1], drive.shape[1])


def _static_forward(library, projected, base, drive, eta_raw, positions, counts, record_tape):
    shape = _shape_of(projected, base, drive)
    output = torch.full((shape.batch, shape.length, shape.heads * shape.head_dim), float("nan"),
                        dtype=torch.bfloat16, device=projected.device)
    tape = None
    if record_tape:
        floats = ctypes.c_size_t()
        assert library.lsso_hip_mixer_tape_floats(ctypes.byref(shape), ctypes.byref(floats)) == 0
        tape = torch.full((floats.value,), float("nan"), dtype=torch.float32, device=projected.device)
    _call_static(library, shape, projected, base, drive, eta_raw, positions, counts, output, tape)
    return output, tape


def _call_static(library, shape, projected, base, drive, eta_raw, positions, counts, output, tape):
    rank = shape.rank
    mode = 0 if positions is None else (2 if positions.dim() == 2 else 1)
    status = library.lsso_hip_mixer_forward_static(
        ctypes.byref(shape),
        projected.data_ptr(),
        base.data_ptr(),
        drive.data_ptr(),
        eta_raw.data_ptr(),
        ctypes.cast(hip._inverse_frequency(rank), ctypes.c_void_p),
        None if positions is None else positions.data_ptr(),
        mode,
        None if counts is None else counts.data_ptr(),
        output.data_ptr(),
        None if tape is None else tape.data_ptr(),
        torch.cuda.current_stream(projected.device).cuda_stream,
    )
    assert status == 0, library.lsso_hip_last_error().decode()


CASES = [
    # (batch, length, heads, rank, head_dim, seed, masked, tape)
    (8, 2000, 8, 32, 32, 1, False, True),
    (3, 257, 2, 32, 32, 2, False, True),
    (4, 1500, 6, 64, 64, 3, True, True),
    (2, 100, 3, 16, 17, 4, True, False),
    (64, 4096, 8, 32, 32, 5, False, False),
    (1, 65, 1, 48, 96, 6, False, True),
]


def test_static_forward_matches_the_workspace_entry_point(library) -> None:
    for batch, length, heads, rank, head_dim, seed, masked, record_tape in CASES:
        print(f"case B={batch} N={length} H={heads} r={rank} d={head_dim} masked={masked}", flush=True)
        projected, base, drive, eta_raw, positions, counts = _inputs(
            batch, length, heads, rank, head_dim, seed, masked)
        expected, expected_tape = hip._mixer_forward(
            projected, base, drive, eta_raw, positions, counts, record_tape)
        out, tape = _static_forward(library, projected, base, drive, eta_raw, positions, counts,
                                    record_tape)
        # A second call in a row on the same scratch.
        again, _ = _static_forward(library, projected, base, drive, eta_raw, positions, counts, False)
        torch.cuda.synchronize()
        assert torch.equal(out, expected)
        assert torch.equal(again, expected)
        if record_tape:
            assert torch.equal(tape, expected_tape)


def test_static_forward_rejects_geometries_beyond_its_scratch(library) -> None:
    shape = hip.MixerShape(64, 65536, 8, 32, 32)
    size = ctypes.c_size_t()
    assert library.lsso_hip_mixer_workspace_bytes(ctypes.byref(shape), 0, ctypes.byref(size)) == 0
    assert size.value > (64 << 20)
    dummy = torch.empty(16, device="cuda")
    status = library.lsso_hip_mixer_forward_static(
        ctypes.byref(shape), dummy.data_ptr(), dummy.data_ptr(), dummy.data_ptr(), dummy.data_ptr(),
        None, None, 0, None, dummy.data_ptr(), None, torch.cuda.current_stream().cuda_stream)
    assert status == -2
    assert "more than the static scratch" in library.lsso_hip_last_error().decode()


def test_static_forward_replays_from_a_captured_graph(library) -> None:
    """Outputs allocated before capture, the device's first static call made
    outside it; every replay, with eager static calls of another geometry
    overwriting the shared array in between, equals the workspace entry."""

    projected, base, drive, eta_raw, positions, counts = _inputs(4, 700, 4, 32, 32, 9)
    expected, _ = hip._mixer_forward(projected, base, drive, eta_raw, positions, counts, False)
    other = _inputs(2, 333, 3, 16, 32, 10, masked=True)
    other_expected, _ = hip._mixer_forward(*other, False)
    shape = _shape_of(projected, base, drive)
    output = torch.empty_like(expected)
    _call_static(library, shape, projected, base, drive, eta_raw, positions, counts, output, None)
    torch.cuda.synchronize()
    assert torch.equal(output, expected)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _call_static(library, shape, projected, base, drive, eta_raw, positions, counts, output, None)
    torch.cuda.synchronize()
    for replay in range(3):
        print(f"replay {replay}", flush=True)
        output.zero_()
        other_out, _ = _static_forward(library, *other, False)
        torch.cuda.synchronize()
        assert torch.equal(other_out, other_expected)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(output, expected), f"replay {replay}"
