"""Independent FP64 restatement of the LSSO mixer -- TEST INFRASTRUCTURE ONLY.

numpy/scipy, no torch, no QR: P = A L^-T with L L^T = A^T A + I, so
Z = L^-1 (A^T C), Y = eta C + A L^-T X.  This is the closed-form identity that
replaces the reference's QR soft frame (lsso/ball/reference.py:411-447;
docs/CUDA_CONTRACT.md: Gram/Cholesky/TRSM schedule).  It cross-checks
oracle/lsso_reference.py (QR) to ~1e-12 and is imported only by tests/.
"""

from __future__ import annotations

import math

import numpy as np
from scipy.linalg import solve_triangular

SOFTPLUS_ONE_OFFSET = math.log(math.expm1(1.0))


def complement(raw: np.ndarray) -> np.ndarray:
    return (1.0 - np.finfo(np.float64).eps) * np.tanh(raw)


def softplus(x: np.ndarray) -> np.ndarray:
    return np.where(x > 20.0, x, np.log1p(np.exp(np.minimum(x, 20.0))))


def mix(projected, base, drive, eta_raw, positions=None, counts=None):
    """projected [B, N, H*R + H*d] -> mixed [B, N, H*d], all FP64."""

    projected = np.asarray(projected, dtype=np.float64)
    base = np.asarray(base, dtype=np.float64)
    drive = np.asarray(drive, dtype=np.float64)
    eta = complement(np.asarray(eta_raw, dtype=np.float64))
    batch, length, width = projected.shape
    heads, rank, _ = base.shape
    head_dim = (width - heads * rank) // heads
    if positions is None:
        positions = np.arange(length, dtype=np.float64) - 0.5 * (length - 1)
    positions = np.broadcast_to(np.asarray(positions, dtype=np.float64), (batch, length))
    if counts is None:
        counts = np.full(batch, float(length))
    counts = np.asarray(counts, dtype=np.float64)
    half = rank // 2
    inv_freq = 10000.0 ** (-np.arange(half, dtype=np.float64) / half)
    angle = positions[:, :, None] * inv_freq[None, None, :]
    cos, sin = np.cos(angle), np.sin(angle)
    out = np.zeros((batch, length, heads * head_dim))
    for b in range(batch):
        root = math.sqrt(counts[b])
        for h in range(heads):
            rel = projected[b, :, h * rank:(h + 1) * rank]
            content = projected[b, :, heads * rank + h * head_dim: heads * rank + (h + 1) * head_dim]
            even, odd = rel[:, 0::2], rel[:, 1::2]
            a = np.empty_like(rel)
            a[:, 0::2] = even * cos[b] - odd * sin[b]
            a[:, 1::2] = even * sin[b] + odd * cos[b]
            a /= root
            lower = np.linalg.cholesky(a.T @ a + np.eye(rank))
            z = solve_triangular(lower, a.T @ content, lower=True)
            theta = base[h] + z @ drive[h] / root
            factor = np.tril(theta, -1) + np.diag(softplus(np.diag(theta) + SOFTPLUS_ONE_OFFSET))
            upper = np.triu(theta, 1)
            system = np.eye(rank) + factor @ factor.T + upper - upper.T
            u = np.linalg.solve(system, z)
            x = 2.0 * u - (1.0 + eta[h]) * z
            m = solve_triangular(lower.T, x, lower=False)
            out[b, :, h * head_dim:(h + 1) * head_dim] = eta[h] * content + a @ m
    return out


def dense_operator(projected, base, drive, eta_raw, b, h, positions=None, counts=None):
    """The N x N token operator T = eta I + P (M - eta I) P^T of one (b, h)
    with M = 2 (I + K)^-1 - I (paper main.tex:357-360; reference test
    tests/core/test_reference.py:410-417).  Used as a brute-force check on
    tiny inputs: mixed[b, :, h-block] == T @ C."""

    projected = np.asarray(projected, dtype=np.float64)
    base = np.asarray(base, dtype=np.float64)
    drive = np.asarray(drive, dtype=np.float64)
    batch, length, width = projected.shape
    heads, rank, _ = base.shape
    head_dim = (width - heads * rank) // heads
    if positions is None:
        positions = np.arange(length, dtype=np.float64) - 0.5 * (length - 1)
    positions = np.broadcast_to(np.asarray(positions, dtype=np.float64), (batch, length))
    count = float(length) if counts is None else float(np.asarray(counts)[b])
    half = rank // 2
    inv_freq = 10000.0 ** (-np.arange(half, dtype=np.float64) / half)
    angle = positions[b, :, None] * inv_freq[None, :]
    rel = projected[b, :, h * rank:(h + 1) * rank]
    content = projected[b, :, heads * rank + h * head_dim: heads * rank + (h + 1) * head_dim]
    a = np.empty_like(rel)
    a[:, 0::2] = rel[:, 0::2] * np.cos(angle) - rel[:, 1::2] * np.sin(angle)
    a[:, 1::2] = rel[:, 0::2] * np.sin(angle) + rel[:, 1::2] * np.cos(angle)
    a /= math.sqrt(count)
    # Frame via the explicit QR of [A; I] with a positive R diagonal.
    q, r = np.linalg.qr(np.vstack((a, np.eye(rank))))
    q = q * np.where(np.diag(r) < 0, -1.0, 1.0)[None, :]
    frame = q[:length]
    z = frame.T @ content
    theta = base[h] + z @ drive[h] / math.sqrt(count)
    factor = np.tril(theta, -1) + np.diag(softplus(np.diag(theta) + SOFTPLUS_ONE_OFFSET))
    upper = np.triu(theta, 1)
    system = np.eye(rank) + factor @ factor.T + upper - upper.T
    reflected = 2.0 * np.linalg.inv(system) - np.eye(rank)
    eta = complement(float(np.asarray(eta_raw)[h]))
    operator = eta * np.eye(length) + frame @ (reflected - eta * np.eye(rank)) @ frame.T
    return operator, content
