"""Input checks (same rules and messages as ``transport/matrix/_validate.py:19-156``).

The value checks (NaN / -inf in the cost, negative marginals) exist twice:
as torch reductions here (:func:`validate_cost`, ``check_sign`` of
:func:`coerce_marginals`), used for inputs the kernels do not read as they
are (float64, host tensors), and as flag bits of the device preparation
pass, which :func:`raise_for_flags` turns into the same exceptions.
"""

from __future__ import annotations

import torch

# flag bits of the device preparation pass (TM_SK_FLAG_* of the C ABI)
FLAG_NAN = 1
FLAG_NEG_INF = 2
FLAG_A_NEG = 4
FLAG_B_NEG = 8
FLAG_ANY_FINITE = 16


def validate_cost_meta(cost: torch.Tensor) -> None:
    """The shape / dtype / device half of :func:`validate_cost` (no sync)."""
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


def validate_cost(cost: torch.Tensor) -> None:
    validate_cost_meta(cost)
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
    check_sign: bool,
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
    if check_sign and (out < 0).any():
        raise ValueError(_negative_message(name))
    return out


def _negative_message(name: str) -> str:
    return f"torchmatch.transport.matrix.solve: {name} must be non-negative"


def raise_for_flags(flags: int, *, cost: bool, marginals: bool) -> None:
    """Raise what the reference's checks raise for the flags of the device
    pass, in the reference's order (cost NaN, cost -inf, a, b)."""
    if cost and flags & FLAG_NAN:
        msg = "torchmatch.transport.matrix.solve: cost contains NaN"
        raise RuntimeError(msg)
    if cost and flags & FLAG_NEG_INF:
        msg = "torchmatch.transport.matrix.solve: cost contains -inf"
        raise RuntimeError(msg)
    if marginals and flags & FLAG_A_NEG:
        raise ValueError(_negative_message("a"))
    if marginals and flags & FLAG_B_NEG:
        raise ValueError(_negative_message("b"))


def coerce_marginals(
    cost: torch.Tensor,
    a: torch.Tensor | None,
    b: torch.Tensor | None,
    *,
    check_sign: bool = True,
) -> tuple[torch.Tensor, torch.Tensor]:
    if cost.ndim == 2:
        n, m = cost.shape
        batch = 1
    else:
        batch, n, m = cost.shape
    a_out = _coerce_one_marginal(cost, a, name="a", dim_label="N", shape=(batch, n),
                                 check_sign=check_sign)
    b_out = _coerce_one_marginal(cost, b, name="b", dim_label="M", shape=(batch, m),
                                 check_sign=check_sign)
    return a_out, b_out


def fuse_mask_into_cost(cost: torch.Tensor, mask: torch.Tensor | None) -> torch.Tensor:
    if mask is None:
        return cost
    return cost.masked_fill(~mask, float("inf"))


def kernel_keep_mask(cost: torch.Tensor, mask: torch.Tensor) -> torch.Tensor | None:
    """``mask`` as the kernels' keep operand: a contiguous bool tensor of
    ``cost``'s shape on its device (True = keep), with the broadcast
    ``masked_fill`` applies.  ``None`` when the mask is one the kernels do not
    take (another dtype or device, a shape that does not broadcast to the
    cost's); the caller then fuses it with :func:`fuse_mask_into_cost`, which
    raises what torch raises for it."""
    if mask.dtype != torch.bool or mask.device != cost.device:
        return None
    if mask.shape != cost.shape:
        try:
            mask = mask.expand(cost.shape)
        except RuntimeError:
            return None
    return mask.contiguous()
