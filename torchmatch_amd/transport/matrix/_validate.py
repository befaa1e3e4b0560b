"""Input checks (same rules and messages as ``transport/matrix/_validate.py:19-156``)."""

from __future__ import annotations

import torch


def validate_cost(cost: torch.Tensor) -> None:
    if cost.ndim not in (2, 3):
        msg = (
            "torchmatch.transport.matrix.solve: cost.ndim must be 2 or 3, "
            f"got {cost.ndim}"
        )
        raise ValueError(msg)
    if cost.dtype not in (torch.float32, torch.float64):
        msg = (
            "torchmatch.transport.matrix.solve: cost.dtype must be float32 "
            f"or float64, got {cost.dtype}"
        )
        raise ValueError(msg)
    if cost.device.type not in ("cpu", "cuda"):
        msg = (
            "torchmatch.transport.matrix.solve: cost.device must be cpu or "
            f"cuda, got {cost.device}"
        )
        raise ValueError(msg)
    if torch.isnan(cost).any():
        msg = "torchmatch.transport.matrix.solve: cost contains NaN"
        raise RuntimeError(msg)
    if (cost == float("-inf")).any():
        msg = "torchmatch.transport.matrix.solve: cost contains -inf"
        raise RuntimeError(msg)


def _coerce_one_marginal(
    cost: torch.Tensor,
    x: torch.Tensor | None,
    *,
    name: str,
    dim_label: str,
    shape: tuple[int, int],
) -> torch.Tensor:
    batch, expected_len = shape
    if x is None:
        fill = 0.0 if expected_len == 0 else 1.0 / expected_len
        return torch.full((batch, expected_len), fill, device=cost.device, dtype=cost.dtype)
    if x.ndim == 1:
        if x.shape != (expected_len,):
            msg = (
                f"torchmatch.transport.matrix.solve: {name} must have shape "
                f"({dim_label},) = ({expected_len},) for 2D cost, "
                f"got {tuple(x.shape)}"
            )
            raise ValueError(msg)
        out = x.to(device=cost.device, dtype=cost.dtype).unsqueeze(0)
        if cost.ndim == 3:
            out = out.expand(batch, expected_len).contiguous()
    else:
        if x.shape != (batch, expected_len):
            msg = (
                f"torchmatch.transport.matrix.solve: {name} must have shape "
                f"(B, {dim_label}) = ({batch}, {expected_len}) for 3D cost, "
                f"got {tuple(x.shape)}"
            )
            raise ValueError(msg)
        out = x.to(device=cost.device, dtype=cost.dtype)
    if (out < 0).any():
        msg = f"torchmatch.transport.matrix.solve: {name} must be non-negative"
        raise ValueError(msg)
    return out


def coerce_marginals(
    cost: torch.Tensor,
    a: torch.Tensor | None,
    b: torch.Tensor | None,
) -> tuple[torch.Tensor, torch.Tensor]:
    if cost.ndim == 2:
        n, m = cost.shape
        batch = 1
    else:
        batch, n, m = cost.shape
    a_out = _coerce_one_marginal(cost, a, name="a", dim_label="N", shape=(batch, n))
    b_out = _coerce_one_marginal(cost, b, name="b", dim_label="M", shape=(batch, m))
    return a_out, b_out


def fuse_mask_into_cost(cost: torch.Tensor, mask: torch.Tensor | None) -> torch.Tensor:
    if mask is None:
        return cost
    return cost.masked_fill(~mask, float("inf"))
