"""Total cost of an assignment (same contract as ``assignment/_cost.py:8-61``)."""

from __future__ import annotations

import torch


def assignment_cost(
    cost: torch.Tensor,
    matches: torch.Tensor,
    *,
    reduction: str = "sum",
) -> torch.Tensor:
    """Sum (or mean, or per-row) cost of a row->col mapping; ``-1`` rows count 0.

    ``cost`` is (N, M) or (B, N, M); ``matches`` is (N,) or (B, N) int64.
    """
    if reduction not in ("sum", "mean", "none"):
        msg = f"assignment_cost: reduction must be 'sum', 'mean' or 'none', got {reduction!r}"
        raise ValueError(msg)
    squeeze = cost.ndim == 2
    if squeeze:
        cost = cost.unsqueeze(0)
        matches = matches.unsqueeze(0)
    valid = matches >= 0
    picked = torch.gather(cost, 2, matches.clamp(min=0).unsqueeze(-1)).squeeze(-1)
    per_row = torch.where(valid, picked, picked.new_zeros(()))
    if reduction == "none":
        out = per_row
    elif reduction == "mean":
        n_matched = valid.sum(dim=-1).clamp(min=1)
        out = per_row.sum(dim=-1) / n_matched.to(per_row.dtype)
    else:
        out = per_row.sum(dim=-1)
    return out.squeeze(0) if squeeze else out
