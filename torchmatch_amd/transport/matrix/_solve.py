"""``solve`` for the cost-matrix face (mirrors ``transport/matrix/_solve.py:98-264``).

``LOG_SINKHORN`` (and ``AUTO``), ``UNBALANCED_SINKHORN`` and
``SINKHORN_DIVERGENCE`` run the gfx950 kernel on device tensors.
``EXACT_EMD`` is a reference backend outside this package and raises
``NotImplementedError``.
"""

from __future__ import annotations

from enum import Enum

import torch

from torchmatch_amd.transport.matrix._sinkhorn import (
    _device_checkable,
    _log_sinkhorn,
    _sinkhorn_divergence,
    _unbalanced_sinkhorn,
)
from torchmatch_amd.transport.matrix._validate import (
    coerce_marginals,
    validate_cost,
    validate_cost_meta,
)

__all__ = ["Backend", "marginal_error", "solve"]


class Backend(str, Enum):
    """Backend names of the reference (``transport/matrix/_solve.py:43-48``)."""

    AUTO = "auto"
    LOG_SINKHORN = "log_sinkhorn"
    SINKHORN_DIVERGENCE = "sinkhorn_divergence"
    UNBALANCED_SINKHORN = "unbalanced_sinkhorn"
    EXACT_EMD = "exact_emd"

    def __str__(self) -> str:
        return self.value


def _coerce_backend(value: Backend | str) -> Backend:
    try:
        return Backend(value)
    except ValueError as err:
        msg = (
            f"torchmatch.transport.matrix.solve: unknown backend {value!r}; "
            f"valid values are {[b.value for b in Backend]}"
        )
        raise ValueError(msg) from err


def solve(  # noqa: PLR0913, PLR0911
    cost: torch.Tensor,
    *,
    backend: Backend | str = Backend.AUTO,
    reg: float = 0.1,
    n_iter: int = 100,
    mask: torch.Tensor | None = None,
    a: torch.Tensor | None = None,
    b: torch.Tensor | None = None,
    scaling: float | None = None,
    rho: float = 1.0,
    cost_aa: torch.Tensor | None = None,
    cost_bb: torch.Tensor | None = None,
    unpack: bool = False,
):
    """Log transport plan of ``cost`` (or ``(log_plan, f, g)`` with ``unpack``)."""
    backend = _coerce_backend(backend)
    validate_cost_meta(cost)
    if backend == Backend.EXACT_EMD:
        validate_cost(cost)
        msg = f"torchmatch_amd.transport.matrix.solve: backend {backend.value!r} is not provided"
        raise NotImplementedError(msg)

    squeeze_batch = cost.ndim == 2
    cost3 = cost.unsqueeze(0) if squeeze_batch else cost
    # the value checks of validate_cost and of the marginals run in the
    # kernels' preparation pass when it reads the values as given (float32 on
    # the device); otherwise torch runs them here, in the reference's order
    try:
        a_, b_ = coerce_marginals(cost3, a, b, check_sign=False)
    except ValueError:
        validate_cost(cost)
        coerce_marginals(cost3, a, b)
        raise
    device_checks = _device_checkable(cost3, a_, b_)
    if not device_checks:
        validate_cost(cost)
        coerce_marginals(cost3, a_, b_)
    cost = cost3
    mask_ = mask.unsqueeze(0) if (squeeze_batch and mask is not None) else mask
    checks = {"mask": mask_, "check_cost": device_checks, "check_marginals": device_checks}

    def _out(x):
        if isinstance(x, tuple):
            return tuple(t.squeeze(0) for t in x) if squeeze_batch else x
        return x.squeeze(0) if squeeze_batch else x

    if backend == Backend.SINKHORN_DIVERGENCE:
        # self-costs are used as given (2-D ones broadcast over the batch)
        result = _sinkhorn_divergence(
            cost, eps=reg, n_iter=n_iter, a=a_, b=b_, scaling=scaling,
            cost_aa=cost_aa, cost_bb=cost_bb, **checks,
        )
        return result.squeeze(0) if squeeze_batch else result

    if backend in (Backend.AUTO, Backend.LOG_SINKHORN):
        res = _log_sinkhorn(
            cost, eps=reg, n_iter=n_iter, a=a_, b=b_, scaling=scaling,
            return_potentials=unpack, **checks,
        )
        return _out(res)

    # UNBALANCED_SINKHORN
    log_plan = _unbalanced_sinkhorn(
        cost, eps=reg, n_iter=n_iter, rho=rho, a=a_, b=b_, scaling=scaling, **checks
    )
    if not unpack:
        return _out(log_plan)
    # potentials from the plan, as transport/matrix/_solve.py:177-213
    mask_a = a_ > 0
    mask_b = b_ > 0
    neg_inf_row = (log_plan == float("-inf")).all(dim=2)
    neg_inf_col = (log_plan == float("-inf")).all(dim=1)
    zero_f = neg_inf_row | ~mask_a
    zero_g = neg_inf_col | ~mask_b
    log_plan_a_safe = torch.where(zero_f[..., None], torch.zeros_like(log_plan), log_plan)
    log_plan_b_safe = torch.where(zero_g[:, None, :], torch.zeros_like(log_plan), log_plan)
    a_safe = torch.where(mask_a, a_, torch.ones_like(a_))
    b_safe = torch.where(mask_b, b_, torch.ones_like(b_))
    f_raw = rho * (torch.logsumexp(log_plan_a_safe, dim=2) - a_safe.log())
    g_raw = rho * (torch.logsumexp(log_plan_b_safe, dim=1) - b_safe.log())
    f = torch.where(zero_f, torch.zeros_like(a_), f_raw)
    g = torch.where(zero_g, torch.zeros_like(b_), g_raw)
    return _out((log_plan, f, g))


def marginal_error(
    log_plan: torch.Tensor,
    a: torch.Tensor,
    b: torch.Tensor,
) -> tuple[float, float]:
    """Max |row sums - a| and |column sums - b| of ``exp(log_plan)``."""
    plan = log_plan.exp()
    row_err = (plan.sum(dim=-1) - a).abs().max().item()
    col_err = (plan.sum(dim=-2) - b).abs().max().item()
    return float(row_err), float(col_err)
