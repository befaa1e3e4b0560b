"""Epsilon schedule (same rules and messages as ``transport/matrix/_schedule.py:21-76``).

``scaling=None`` gives ``n_iter`` copies of ``reg``; otherwise a geometric
decay from ``max(0.5 * max finite cost, reg)`` by ``scaling`` per step,
clamped at ``reg``.
"""

from __future__ import annotations

import torch


def check_schedule_args(*, reg: float, n_iter: int, scaling: float | None) -> None:
    if reg <= 0:
        msg = f"torchmatch.transport.matrix.solve: reg must be positive, got {reg}"
        raise ValueError(msg)
    if n_iter < 1:
        msg = f"torchmatch.transport.matrix.solve: n_iter must be >= 1, got {n_iter}"
        raise ValueError(msg)
    if scaling is not None and not (0.0 < scaling < 1.0):
        msg = (
            "torchmatch.transport.matrix.solve: scaling must be in (0, 1), "
            f"got {scaling}"
        )
        raise ValueError(msg)


def schedule_from_max(
    *,
    reg: float,
    n_iter: int,
    scaling: float | None,
    max_finite: float | None,
) -> list[float]:
    """The schedule given the largest finite cost (``None``: no finite entry),
    which the device preparation pass measures in the same sweep that
    validates the cost."""
    check_schedule_args(reg=reg, n_iter=n_iter, scaling=scaling)
    if scaling is None:
        return [reg] * n_iter
    initial = reg if max_finite is None else max(0.5 * max_finite, reg)
    schedule: list[float] = []
    current = initial
    for _ in range(n_iter):
        schedule.append(current)
        current = reg if current <= reg else max(current * scaling, reg)
    return schedule


def build_eps_schedule(
    *,
    cost: torch.Tensor,
    reg: float,
    n_iter: int,
    scaling: float | None,
) -> list[float]:
    check_schedule_args(reg=reg, n_iter=n_iter, scaling=scaling)
    max_finite = None
    if scaling is not None:
        finite = cost[torch.isfinite(cost)]
        if finite.numel() != 0:
            max_finite = finite.max().item()
    return schedule_from_max(reg=reg, n_iter=n_iter, scaling=scaling, max_finite=max_finite)
