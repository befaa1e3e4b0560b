"""Seeded synthetic inputs for the benchmark configurations (CPU tensors).

Every generator uses a CPU ``torch.Generator`` so the bytes are the same on
any machine with the same torch build; :func:`sha256` fingerprints them.

* ``jv_uniform(B, N, M)``        -- C1 (8,16,16) and C2 (1024,64,64):
  ``torch.rand`` i.i.d. U[0,1) float32.
* ``jv_rect_masked()``           -- C3 (64,512,768): squared Euclidean
  distances between N(0,1) point sets in D=16, + 1e-6*U[0,1) jitter, then
  +inf on a U[0,1) < 0.2 draw.
* ``sinkhorn_points(B, N, M, D)`` -- C4/C5 cost: squared Euclidean distances
  between N(0,I) clouds, divided by the global max, built in row chunks.
* ``dirichlet(B, N, total)``     -- marginals: normalised Exp(1) draws.
* ``integer_tied`` / ``gated_sparse`` -- tie-heavy and +inf-heavy JV inputs
  following the reference's ``tests/_costgen.py:75-96``.
"""

from __future__ import annotations

import hashlib

import torch


def _gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def sha256(t: torch.Tensor) -> str:
    return hashlib.sha256(t.detach().cpu().contiguous().numpy().tobytes()).hexdigest()


def jv_uniform(B: int, N: int, M: int, seed: int = 0) -> torch.Tensor:
    return torch.rand(B, N, M, dtype=torch.float32, generator=_gen(seed))


def jv_rect_masked(
    B: int = 64, N: int = 512, M: int = 768, D: int = 16, p_inf: float = 0.2, seed: int = 0
) -> torch.Tensor:
    g = _gen(seed)
    x = torch.randn(B, N, D, dtype=torch.float32, generator=g)
    y = torch.randn(B, M, D, dtype=torch.float32, generator=g)
    c = torch.empty(B, N, M, dtype=torch.float32)
    for b in range(B):
        c[b] = ((x[b, :, None, :] - y[b, None, :, :]) ** 2).sum(-1)
    c += 1e-6 * torch.rand(B, N, M, dtype=torch.float32, generator=g)
    c[torch.rand(B, N, M, generator=g) < p_inf] = float("inf")
    return c


def integer_tied(B: int, N: int, M: int, seed: int = 0, hi: int = 8) -> torch.Tensor:
    return torch.randint(0, hi, (B, N, M), generator=_gen(seed)).to(torch.float32)


def gated_sparse(B: int, n: int, seed: int = 0) -> torch.Tensor:
    """About 70% +inf cells with a planted finite permutation (halved costs)."""
    g = _gen(seed)
    cost = torch.rand(B, n, n, dtype=torch.float32, generator=g)
    out = torch.empty_like(cost)
    rows = torch.arange(n)
    for b in range(B):
        perm = torch.randperm(n, generator=g)
        prob = torch.full((n, n), 0.7)
        prob[rows, perm] = 0.0
        mask = torch.rand(n, n, generator=g) < prob
        cb = cost[b].masked_fill(mask, float("inf"))
        cb[rows, perm] *= 0.5
        out[b] = cb
    return out


def sinkhorn_points(B: int, N: int, M: int, D: int = 8, seed: int = 0,
                    chunk: int = 1024) -> torch.Tensor:
    g = _gen(seed)
    x = torch.randn(B, N, D, dtype=torch.float32, generator=g)
    y = torch.randn(B, M, D, dtype=torch.float32, generator=g)
    c = torch.empty(B, N, M, dtype=torch.float32)
    for b in range(B):
        for i0 in range(0, N, chunk):
            xi = x[b, i0:i0 + chunk]
            c[b, i0:i0 + chunk] = ((xi[:, None, :] - y[b, None, :, :]) ** 2).sum(-1)
    c /= c.max()
    return c


def dirichlet(B: int, N: int, total: float = 1.0, seed: int = 0) -> torch.Tensor:
    e = torch.empty(B, N, dtype=torch.float32).exponential_(1.0, generator=_gen(seed))
    return e / e.sum(dim=1, keepdim=True) * total


def uniform_marginal(B: int, N: int) -> torch.Tensor:
    return torch.full((B, N), 1.0 / N, dtype=torch.float32)
