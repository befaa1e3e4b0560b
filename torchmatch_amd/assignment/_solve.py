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
    if unpack:
        # the device unpack, as the reference's native-unpack path
        # (assignment/_solve.py:207-209) returns the CPU op's tuple; a 2-D
        # problem is a batch of one, trimmed of the -1 padding as the
        # reference's 2-D unpack returns it (:124-164)
        matches, ur, uc, nm = torch.ops.assignment.jonker_dense_batch_unpacked(
            batch.contiguous())
        if not squeeze:
            return matches, ur, uc, nm
        k = int(nm[0].item())
        return matches[0, :k], ur[0, : n - k], uc[0, : m - k]
    packed = torch.ops.assignment.jonker_dense_batch(batch.contiguous())
    return packed[0] if squeeze else packed


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
