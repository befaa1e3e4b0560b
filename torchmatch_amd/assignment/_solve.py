"""Dispatcher over the gfx950 assignment op (mirrors ``assignment/_solve.py``).

Routing on a ROCm device (device type ``"cuda"``):

* 3-D ``(B, N, M)`` with ``max(N, M) <= torch.ops.assignment`` kernel limit
  -> ``torch.ops.assignment.jonker_dense_batch`` (reference: square K <= 64
  only, ``_solve.py:95-97,187-199``; the gfx950 kernel also takes rectangular
  batches, whose results follow the reference CPU op);
* 2-D ``(N, M)`` -> the same op on a batch of one.

CPU tensors are not handled here: the reference's CPU extension owns them.
The reference's other backends (munkres, lawler, greedy) are outside this
package and raise ``NotImplementedError`` when requested explicitly.
"""

from __future__ import annotations

from enum import Enum

import torch

from torchmatch_amd._native import jv_max_k

__all__ = ["Backend", "resolve_backend", "solve"]


class Backend(str, Enum):
    """Backend names of the reference (``assignment/_solve.py:25-30``)."""

    AUTO = "auto"
    JONKER = "jonker"
    MUNKRES = "munkres"
    LAWLER = "lawler"
    GREEDY = "greedy"

    def __str__(self) -> str:  # StrEnum behaviour on Python 3.10
        return self.value


_PROVIDED = (Backend.AUTO, Backend.JONKER)


def _coerce_backend(value: Backend | str) -> Backend:
    try:
        return Backend(value)
    except ValueError as err:
        msg = (
            f"torchmatch.assignment.solve: unknown backend {value!r}; "
            f"valid values are {[b.value for b in Backend]}"
        )
        raise ValueError(msg) from err


def _validate(cost: torch.Tensor) -> None:
    """Same checks and messages as ``assignment/_solve.py:215-244``."""
    if cost.ndim not in (2, 3):
        msg = f"torchmatch.assignment.solve: cost.ndim must be 2 or 3, got {cost.ndim}"
        raise ValueError(msg)
    if cost.dtype not in (torch.float32, torch.float64):
        msg = (
            "torchmatch.assignment.solve: cost.dtype must be float32 or float64, "
            f"got {cost.dtype}"
        )
        raise ValueError(msg)
    if cost.device.type not in ("cpu", "cuda"):
        msg = (
            "torchmatch.assignment.solve: cost.device must be cpu or cuda, "
            f"got {cost.device}"
        )
        raise ValueError(msg)
    if cost.device.type != "cuda":
        msg = (
            "torchmatch_amd.assignment.solve: this package runs on ROCm devices only; "
            "CPU tensors belong to the reference CPU extension"
        )
        raise ValueError(msg)
    if torch.isnan(cost).any():
        msg = "torchmatch.assignment.solve: cost contains NaN"
        raise RuntimeError(msg)
    if (cost == float("-inf")).any():
        msg = "torchmatch.assignment.solve: cost contains -inf"
        raise RuntimeError(msg)


def _unpack_packed_3d(
    packed: torch.Tensor, m: int
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """(matches, unmatched_rows, unmatched_cols, n_matched), as ``_solve.py:124-164``."""
    b, n = packed.shape
    device = packed.device
    matched_mask = packed >= 0
    n_matched = matched_mask.sum(dim=-1)
    match_order = torch.argsort((~matched_mask).long(), dim=-1, stable=True)
    row_idx = torch.arange(n, device=device).expand(b, n)
    sorted_rows = torch.gather(row_idx, 1, match_order)
    sorted_cols = torch.gather(packed, 1, match_order)
    matches = torch.stack([sorted_rows, sorted_cols], dim=-1)
    unmatched_order = torch.argsort(matched_mask.long(), dim=-1, stable=True)
    unmatched_rows = torch.gather(row_idx, 1, unmatched_order)
    col_mask = torch.zeros(b, m, dtype=torch.bool, device=device)
    col_mask.scatter_(1, packed.clamp(min=0), matched_mask)
    col_order = torch.argsort(col_mask.long(), dim=-1, stable=True)
    col_range = torch.arange(m, device=device).expand(b, m)
    unmatched_cols = torch.gather(col_range, 1, col_order)
    return matches, unmatched_rows, unmatched_cols, n_matched


def _unpack_packed(packed: torch.Tensor, m: int) -> tuple[torch.Tensor, ...]:
    if packed.ndim == 1:
        matches3, ur3, uc3, n_matched = _unpack_packed_3d(packed.unsqueeze(0), m)
        k = int(n_matched.item())
        n = packed.size(0)
        return matches3[0, :k], ur3[0, : n - k], uc3[0, : m - k]
    return _unpack_packed_3d(packed, m)


def _dispatch_jonker(cost: torch.Tensor, *, unpack: bool):
    squeeze = cost.ndim == 2
    batch = cost.unsqueeze(0) if squeeze else cost
    n, m = batch.shape[1], batch.shape[2]
    if max(n, m) > jv_max_k():
        msg = (
            "torchmatch_amd.assignment.solve: the gfx950 batched JV kernel requires "
            f"max(N, M) <= {jv_max_k()}, got shape {tuple(cost.shape)}"
        )
        raise ValueError(msg)
    if unpack and not squeeze:
        # the device unpack, as the reference's native-unpack path
        # (assignment/_solve.py:207-209) returns the CPU op's tuple
        return torch.ops.assignment.jonker_dense_batch_unpacked(batch.contiguous())
    packed = torch.ops.assignment.jonker_dense_batch(batch.contiguous())
    if squeeze:
        packed = packed[0]
    return _unpack_packed(packed, m) if unpack else packed


def solve(
    cost: torch.Tensor,
    *,
    backend: Backend | str = Backend.AUTO,
    unpack: bool = False,
) -> torch.Tensor | tuple[torch.Tensor, ...]:
    """Solve one (N, M) or a batch (B, N, M) of assignment problems on device."""
    backend = _coerce_backend(backend)
    _validate(cost)
    if backend not in _PROVIDED:
        msg = f"torchmatch_amd.assignment.solve: backend {backend.value!r} is not provided"
        raise NotImplementedError(msg)
    return _dispatch_jonker(cost, unpack=unpack)


def resolve_backend(cost: torch.Tensor, *, backend: Backend | str = Backend.AUTO) -> str:
    """Name of the ``torch.ops.assignment`` op :func:`solve` would call."""
    backend = _coerce_backend(backend)
    if backend not in _PROVIDED:
        return backend.value
    return "jonker_dense_batch"
