"""CPU restatement of torchmatch's log-domain Sinkhorn (TEST INFRASTRUCTURE ONLY).

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg
may import this module; the product never does.

The reference computes Sinkhorn with plain torch calls, so the restatement
uses the same torch calls in the same order (on CPU tensors, so it runs on
the same torch build as the tests):

* :func:`log_sinkhorn_plan` follows ``transport/matrix/_log_sinkhorn.py:33-44``
  (masks, -80 stand-in) and ``:136-221`` (iteration, plan, potentials);
* :func:`unbalanced_sinkhorn_plan` follows
  ``transport/matrix/_unbalanced_sinkhorn.py:30-103``;
* :func:`eps_schedule` follows ``transport/matrix/_schedule.py:21-76``.

``dtype`` may be float64 to measure how far float32 itself drifts.

Pinning (tests/test_oracle_sinkhorn.py): the 1x1 unbalanced closed form
``log pi = (rho (log a + log b) - c) / (eps + 2 rho)``; a uniform cost gives
the uniform plan; balanced marginals converge; +inf cells give -inf plan
cells and all-+inf rows give -inf rows without NaN; an independent float64
numpy implementation (scipy.special.logsumexp) of the same recurrence.
"""

from __future__ import annotations

import torch

SAFE_FILL = -80.0  # _log_sinkhorn.py:33


def eps_schedule(cost: torch.Tensor, reg: float, n_iter: int, scaling: float | None) -> list[float]:
    if reg <= 0:
        raise ValueError(f"reg must be positive, got {reg}")
    if n_iter < 1:
        raise ValueError(f"n_iter must be >= 1, got {n_iter}")
    if scaling is None:
        return [reg] * n_iter
    finite = cost[torch.isfinite(cost)]
    initial = reg if finite.numel() == 0 else max(0.5 * finite.max().item(), reg)
    out: list[float] = []
    cur = initial
    for _ in range(n_iter):
        out.append(cur)
        cur = reg if cur <= reg else max(cur * scaling, reg)
    return out


def _masks(cost: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    is_inf = cost == float("inf")
    return is_inf.all(dim=-1), is_inf.all(dim=-2)


def _iterate(cost, a, b, schedule, rho: float | None):
    b_size, rows, cols = cost.shape
    log_mu = a.log()
    log_nu = b.log()
    inf_row, inf_col = _masks(cost)
    log_u = torch.zeros(b_size, rows, dtype=cost.dtype)
    log_v = torch.zeros(b_size, cols, dtype=cost.dtype)
    for step_eps in schedule:
        log_kernel = -cost / step_eps
        krs = torch.where(inf_row[:, :, None], SAFE_FILL, log_kernel)
        kcs = torch.where(inf_col[:, None, :], SAFE_FILL, log_kernel)
        lse_col = torch.logsumexp(krs + log_v[:, None, :], dim=2)
        lse_col = torch.where(inf_row, float("-inf"), lse_col)
        if rho is None:
            log_u = torch.where(lse_col.isfinite(), log_mu - lse_col, log_u)
        else:
            damping = 1.0 / (1.0 + step_eps / rho)
            log_u = torch.where(lse_col.isfinite(), damping * (log_mu - lse_col), log_u)
        lse_row = torch.logsumexp(kcs + log_u[:, :, None], dim=1)
        lse_row = torch.where(inf_col, float("-inf"), lse_row)
        if rho is None:
            log_v = torch.where(lse_row.isfinite(), log_nu - lse_row, log_v)
        else:
            damping = 1.0 / (1.0 + step_eps / rho)
            log_v = torch.where(lse_row.isfinite(), damping * (log_nu - lse_row), log_v)
    log_kernel = -cost / schedule[-1]
    log_plan = log_u[:, :, None] + log_kernel + log_v[:, None, :]
    return log_plan, log_u, log_v


def log_sinkhorn_plan(cost, *, eps, n_iter, a, b, scaling=None, dtype=None):
    """Returns ``(log_plan, f, g, log_u, log_v)`` on CPU."""
    dtype = dtype or cost.dtype
    cost = cost.detach().cpu().to(dtype)
    a = a.detach().cpu().to(dtype)
    b = b.detach().cpu().to(dtype)
    schedule = eps_schedule(cost, eps, n_iter, scaling)
    log_plan, log_u, log_v = _iterate(cost, a, b, schedule, None)
    final_eps = schedule[-1]
    return log_plan, -final_eps * log_u, -final_eps * log_v, log_u, log_v


def unbalanced_sinkhorn_plan(cost, *, eps, n_iter, rho, a, b, scaling=None, dtype=None):
    """Returns ``(log_plan, log_u, log_v)`` on CPU."""
    if rho <= 0:
        raise ValueError("rho must be positive")
    dtype = dtype or cost.dtype
    cost = cost.detach().cpu().to(dtype)
    a = a.detach().cpu().to(dtype)
    b = b.detach().cpu().to(dtype)
    schedule = eps_schedule(cost, eps, n_iter, scaling)
    return _iterate(cost, a, b, schedule, float(rho))
