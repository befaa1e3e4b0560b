"""Epsilon schedule (same rules and messages as ``transport/matrix/_schedule.py:21-76``).

``scaling=None`` gives ``n_iter`` copies of ``reg``; otherwise a geometric
decay from ``max(0.5 * max finite cost, reg)`` by ``scaling`` per step,
clamped at ``reg``.
"""

from __future__ import annotations

import torch


def build_eps_schedule(
    *,
    cost: torch.Tensor,
    reg: float,
    n_iter: int,
    scaling: float | None,
) -> list[float]:
    if reg <= 0:
        msg = f"torchmatch.transport.matrix.solve: reg must be positive, got {reg}"
        raise ValueError(msg)
    if n_iter < 1:
        msg = f"torchmatch.transport.matrix.solve: n_iter must be >= 1, got {n_iter}"
        raise ValueError(msg)
    if scaling is None:
        return [reg] * n_iter
    if not (0.0 < scaling < 1.0):
        msg = (
            "torchmatch.transport.matrix.solve: scaling must be in (0, 1), "
            f"got {scaling}"
        )
        raise ValueError(msg)
    finite = cost[torch.isfinite(cost)]
    initial = reg if finite.numel() == 0 else max(0.5 * finite.max().item(), reg)
    schedule: list[float] = []
    current = initial
    for _ in range(n_iter):
        schedule.append(current)
        current = reg if current <= reg else max(current * scaling, reg)
    return schedule
