"""Device log-domain Sinkhorn (balanced and unbalanced) behind the reference's ops.

Python surface mirrored from the reference:

* :func:`log_sinkhorn_plan`  -- ``transport/matrix/_log_sinkhorn.py:136-221``
* :func:`unbalanced_sinkhorn_plan` -- ``transport/matrix/_unbalanced_sinkhorn.py:30-103``
* :func:`sinkhorn_divergence` -- ``transport/matrix/_sinkhorn_divergence.py:56-128``
* ops ``transport::log_sinkhorn`` (``_log_sinkhorn.py:224-266``),
  ``transport::unbalanced_sinkhorn`` (``_unbalanced_sinkhorn.py:106-153``) and
  ``transport::sinkhorn_divergence`` (``_sinkhorn_divergence.py:131-173``),
  same schemas (inferred from the same Python signatures), same fakes.

The work runs in the gfx950 kernels of ``csrc/sinkhorn.hip`` via two private
ops: ``torchmatch_amd::sinkhorn_prepare`` (one pass over cost, mask and
marginals: the log kernel for the first step, the all-+inf row / column
flags, and what the reference's validation and schedule read from the cost,
NaN / -inf, negative marginals, the largest finite cost, fetched with one
host synchronisation) and ``torchmatch_amd::sinkhorn_iterate``.  A mask is
fused in the kernels (the fused cost is never materialised).  This module
raises the reference's errors from the returned flags, builds the epsilon
schedule and shapes the results.  Like the reference, the iteration runs in
the cost's dtype: float32 costs take the kernels above; float64 costs are
validated by torch and solved by the float64 kernels of
``csrc/sinkhorn64.hip`` (``torchmatch_amd::sinkhorn_f64``).  Device
tensors only: there is no host or torch-eager fallback.  Autograd through the
kernel is not provided (the reference's ``solve`` differentiates through
torch eager code instead).
"""

from __future__ import annotations

import torch

from torchmatch_amd._loader import _has_op
from torchmatch_amd._loader import load as _load
from torchmatch_amd.transport.matrix._schedule import build_eps_schedule, schedule_from_max
from torchmatch_amd.transport.matrix._validate import (
    FLAG_ANY_FINITE,
    fuse_mask_into_cost,
    kernel_keep_mask,
    raise_for_flags,
    validate_cost,
    validate_cost_meta,
)

_load()

_LIBS: list[object] = []


def _require_device(cost: torch.Tensor, a: torch.Tensor, b: torch.Tensor, who: str) -> None:
    if cost.device.type != "cuda" or a.device.type != "cuda" or b.device.type != "cuda":
        msg = (
            f"{who}: torchmatch_amd runs Sinkhorn on ROCm devices only "
            f"(got cost on {cost.device}, a on {a.device}, b on {b.device})"
        )
        raise ValueError(msg)
    if cost.requires_grad or a.requires_grad or b.requires_grad:
        msg = f"{who}: autograd through the gfx950 Sinkhorn kernel is not supported"
        raise NotImplementedError(msg)


def _device_checkable(cost: torch.Tensor, a: torch.Tensor, b: torch.Tensor) -> bool:
    """True when the device pass can run the value checks itself: it reads the
    float32 cost as given (a float64 cost is checked in float64 by torch)."""
    return (
        cost.dtype == torch.float32
        and cost.device.type == "cuda"
        and a.device.type == "cuda"
        and b.device.type == "cuda"
        and not (cost.requires_grad or a.requires_grad or b.requires_grad)
    )


def _torch_marginal_signs(a: torch.Tensor, b: torch.Tensor) -> None:
    raise_for_flags(
        (4 if bool((a < 0).any()) else 0) | (8 if bool((b < 0).any()) else 0),
        cost=False, marginals=True,
    )


def _device_solve(  # noqa: PLR0913
    cost: torch.Tensor,
    a: torch.Tensor,
    b: torch.Tensor,
    *,
    eps: float,
    n_iter: int,
    scaling: float | None,
    rho: float,
    who: str,
    mask: torch.Tensor | None = None,
    check_cost: bool = False,
    check_marginals: bool = False,
    before_schedule=None,
    write_plan: bool = True,
):
    """One solve: the preparation pass (mask fusion, validation, largest
    finite cost), the schedule, then the iteration.  Returns
    ``(schedule, log_plan, log_u, log_v)``; log_plan is None without
    ``write_plan``.

    The checks raise in the reference's order: cost NaN / -inf
    (``_validate.py:58-63``), negative marginals (``:108-110``), then
    ``before_schedule`` (the callers' rho checks), then the schedule's own
    argument checks (``_schedule.py:45-66``).  On the device path all value
    checks and the schedule's largest finite cost come from one pass and one
    host synchronisation; the synchronisation is skipped when nothing needs
    it (no checks and no epsilon scaling)."""
    keep = None
    if mask is not None and _device_checkable(cost, a, b):
        keep = kernel_keep_mask(cost, mask)
    device_checks = _device_checkable(cost, a, b) and (mask is None or keep is not None)
    if not device_checks:
        if check_cost:
            validate_cost(cost)
        if check_marginals:
            _torch_marginal_signs(a, b)
        cost = fuse_mask_into_cost(cost, mask)
        if before_schedule is not None:
            before_schedule()
        schedule = build_eps_schedule(cost=cost, reg=eps, n_iter=n_iter, scaling=scaling)
        b_size, rows, cols = cost.shape
        if b_size == 0:
            plan = cost.new_empty(b_size, rows, cols) if write_plan else None
            return schedule, plan, cost.new_empty(b_size, rows), cost.new_empty(b_size, cols)
        _require_device(cost, a, b, who)
        if cost.dtype == torch.float64:
            # the reference iterates in the cost's dtype: float64 kernels
            log_plan, log_u, log_v = torch.ops.torchmatch_amd.sinkhorn_f64(
                cost.contiguous(), a.to(torch.float64).contiguous(),
                b.to(torch.float64).contiguous(), schedule, float(rho), write_plan)
            return schedule, (log_plan if write_plan else None), log_u, log_v
    c32 = cost.to(torch.float32).contiguous()
    a32 = a.to(torch.float32).contiguous()
    b32 = b.to(torch.float32).contiguous()
    if device_checks:
        # K for the first step is written by the same pass when the schedule
        # is known before it (no scaling)
        k_eps = float(eps) if (scaling is None and eps > 0 and n_iter >= 1) else 0.0
        read = check_cost or check_marginals or scaling is not None
        ws, stats = torch.ops.torchmatch_amd.sinkhorn_prepare(c32, keep, a32, b32, k_eps, read)
        max_finite = None
        if read:
            flags = int(stats[0].item())
            raise_for_flags(flags, cost=check_cost, marginals=check_marginals)
            if flags & FLAG_ANY_FINITE:
                max_finite = float(stats[1].item())
        if before_schedule is not None:
            before_schedule()
        schedule = schedule_from_max(reg=eps, n_iter=n_iter, scaling=scaling,
                                     max_finite=max_finite)
    else:
        k_eps = float(schedule[0])
        ws, _ = torch.ops.torchmatch_amd.sinkhorn_prepare(c32, None, a32, b32, k_eps, False)
    log_plan, log_u, log_v = torch.ops.torchmatch_amd.sinkhorn_iterate(
        c32, keep, ws, schedule, float(rho), k_eps, write_plan
    )
    return schedule, (log_plan if write_plan else None), log_u, log_v


def _log_sinkhorn(  # noqa: PLR0913
    cost, *, eps, n_iter, a, b, scaling=None, return_potentials=False, mask=None,
    check_cost=False, check_marginals=False,
):
    schedule, log_plan, log_u, log_v = _device_solve(
        cost, a, b, eps=eps, n_iter=n_iter, scaling=scaling, rho=0.0, who="log_sinkhorn",
        mask=mask, check_cost=check_cost, check_marginals=check_marginals,
    )
    log_plan = log_plan.to(cost.dtype)
    if return_potentials:
        final_eps = schedule[-1]
        f = (-final_eps * log_u).to(cost.dtype)
        g = (-final_eps * log_v).to(cost.dtype)
        return log_plan, f, g
    return log_plan


def log_sinkhorn_plan(  # noqa: PLR0913
    cost: torch.Tensor,
    *,
    eps: float,
    n_iter: int,
    a: torch.Tensor,
    b: torch.Tensor,
    scaling: float | None = None,
    return_potentials: bool = False,
):
    """Log plan (B, N, M), or ``(log_plan, f, g)`` with ``f = -eps_final * log_u``."""
    return _log_sinkhorn(cost, eps=eps, n_iter=n_iter, a=a, b=b, scaling=scaling,
                         return_potentials=return_potentials)


def _rho_check(rho: float, msg: str):
    def check() -> None:
        if rho <= 0:
            raise ValueError(msg)
    return check


def _solve_rho_message(rho: float) -> str:
    return (
        "torchmatch.transport.matrix.solve: rho must be positive for "
        f"UNBALANCED_SINKHORN, got {rho}"
    )


def _unbalanced_sinkhorn(  # noqa: PLR0913
    cost, *, eps, n_iter, rho, a, b, scaling=None, mask=None, check_cost=False,
    check_marginals=False,
):
    _, log_plan, _, _ = _device_solve(
        cost, a, b, eps=eps, n_iter=n_iter, scaling=scaling, rho=float(rho),
        who="unbalanced_sinkhorn", mask=mask, check_cost=check_cost,
        check_marginals=check_marginals,
        before_schedule=_rho_check(rho, _solve_rho_message(rho)),
    )
    return log_plan.to(cost.dtype)


def unbalanced_sinkhorn_plan(  # noqa: PLR0913
    cost: torch.Tensor,
    *,
    eps: float,
    n_iter: int,
    rho: float,
    a: torch.Tensor,
    b: torch.Tensor,
    scaling: float | None = None,
) -> torch.Tensor:
    """Unbalanced (KL-penalised) log plan (B, N, M)."""
    if rho <= 0:
        raise ValueError(_solve_rho_message(rho))
    return _unbalanced_sinkhorn(cost, eps=eps, n_iter=n_iter, rho=rho, a=a, b=b,
                                scaling=scaling)


def _potentials(cost, a, b, eps, n_iter, scaling, **checks):
    """(f, g) of ``log_sinkhorn_plan(..., return_potentials=True)`` without
    writing the plan (the divergence reads only the potentials)."""
    schedule, _, log_u, log_v = _device_solve(
        cost, a, b, eps=eps, n_iter=n_iter, scaling=scaling, rho=0.0,
        who="sinkhorn_divergence", write_plan=False, **checks,
    )
    final_eps = schedule[-1]
    return (-final_eps * log_u).to(cost.dtype), (-final_eps * log_v).to(cost.dtype)


def _expand_self_cost(c_self, ref: torch.Tensor, b: int, k: int) -> torch.Tensor:
    """``c_self`` broadcast to (b, k, k), or zeros (``_sinkhorn_divergence.py:44-53``)."""
    if c_self is None:
        return torch.zeros(b, k, k, device=ref.device, dtype=ref.dtype)
    c_self = c_self.to(device=ref.device, dtype=ref.dtype)
    if c_self.ndim == 2:
        c_self = c_self.unsqueeze(0)
    return c_self.expand(b, -1, -1)


def _sinkhorn_divergence(  # noqa: PLR0913
    cost, *, eps, n_iter, a, b, scaling=None, cost_aa=None, cost_bb=None, mask=None,
    check_cost=False, check_marginals=False,
):
    batch = cost.size(0)
    n = a.size(-1)
    m = b.size(-1)

    def ot(c, p, q, **checks):
        f, g = _potentials(c, p, q, eps, n_iter, scaling, **checks)
        return (p * f).sum(dim=-1) + (q * g).sum(dim=-1)

    ot_ab = ot(cost, a, b, mask=mask, check_cost=check_cost, check_marginals=check_marginals)
    ot_aa = ot(_expand_self_cost(cost_aa, cost, batch, n), a, a)
    ot_bb = ot(_expand_self_cost(cost_bb, cost, batch, m), b, b)
    return -(ot_ab - 0.5 * ot_aa - 0.5 * ot_bb)


def sinkhorn_divergence(  # noqa: PLR0913
    cost: torch.Tensor,
    *,
    eps: float,
    n_iter: int,
    a: torch.Tensor,
    b: torch.Tensor,
    scaling: float | None = None,
    cost_aa: torch.Tensor | None = None,
    cost_bb: torch.Tensor | None = None,
) -> torch.Tensor:
    """``S_eps(a, b) = OT(a, b) - OT(a, a)/2 - OT(b, b)/2``, each OT the dual
    value ``<a, f> + <b, g>`` of a converged kernel run (B,).

    With ``f = -eps * log_u`` the dual inner product is minus the OT cost, so
    the combination is negated, as ``_sinkhorn_divergence.py:125-128`` does.
    Missing self-costs are zero matrices (the entropic-bias-only variant).
    """
    return _sinkhorn_divergence(cost, eps=eps, n_iter=n_iter, a=a, b=b, scaling=scaling,
                                cost_aa=cost_aa, cost_bb=cost_bb)


def _check_op_cost(cost: torch.Tensor, op: str, hint: str = "") -> None:
    """``validate_cost`` then ``cost.ndim == 3`` as the ops check them; the
    value half of validate_cost is left to the device pass for 3-D costs."""
    if cost.ndim != 3:
        validate_cost(cost)
        msg = f"torch.ops.transport.{op}: cost.ndim must be 3, got {cost.ndim}{hint}"
        raise ValueError(msg)
    validate_cost_meta(cost)


# ---- op registrations ------------------------------------------------------------


def _log_sinkhorn_impl(  # noqa: PLR0913
    cost: torch.Tensor,
    eps: float,
    n_iter: int,
    a: torch.Tensor,
    b: torch.Tensor,
    mask: torch.Tensor | None = None,
    scaling: float | None = None,
) -> torch.Tensor:
    _check_op_cost(
        cost, "log_sinkhorn",
        ". Call torchmatch.transport.matrix.solve(...) for 2-D ergonomic dispatch.",
    )
    return _log_sinkhorn(cost, eps=eps, n_iter=n_iter, a=a, b=b, scaling=scaling, mask=mask,
                         check_cost=True)


def _log_sinkhorn_fake(  # noqa: PLR0913
    cost: torch.Tensor,
    eps: float,
    n_iter: int,
    a: torch.Tensor,
    b: torch.Tensor,
    mask: torch.Tensor | None = None,
    scaling: float | None = None,
) -> torch.Tensor:
    del eps, n_iter, a, b, mask, scaling
    torch._check(cost.dim() == 3, lambda: "cost must be 3D (B, N, M)")
    return cost.new_empty(cost.size(0), cost.size(1), cost.size(2))


def _unbalanced_sinkhorn_impl(  # noqa: PLR0913
    cost: torch.Tensor,
    eps: float,
    n_iter: int,
    rho: float,
    a: torch.Tensor,
    b: torch.Tensor,
    mask: torch.Tensor | None = None,
    scaling: float | None = None,
) -> torch.Tensor:
    _check_op_cost(cost, "unbalanced_sinkhorn")
    _, log_plan, _, _ = _device_solve(
        cost, a, b, eps=eps, n_iter=n_iter, scaling=scaling, rho=float(rho),
        who="unbalanced_sinkhorn", mask=mask, check_cost=True,
        before_schedule=_rho_check(
            rho, "torch.ops.transport.unbalanced_sinkhorn: rho must be positive"
        ),
    )
    return log_plan.to(cost.dtype)


def _unbalanced_sinkhorn_fake(  # noqa: PLR0913
    cost: torch.Tensor,
    eps: float,
    n_iter: int,
    rho: float,
    a: torch.Tensor,
    b: torch.Tensor,
    mask: torch.Tensor | None = None,
    scaling: float | None = None,
) -> torch.Tensor:
    del eps, n_iter, rho, a, b, mask, scaling
    torch._check(cost.dim() == 3, lambda: "cost must be 3D (B, N, M)")
    return cost.new_empty(cost.size(0), cost.size(1), cost.size(2))


def _sinkhorn_divergence_impl(  # noqa: PLR0913
    cost: torch.Tensor,
    eps: float,
    n_iter: int,
    a: torch.Tensor,
    b: torch.Tensor,
    mask: torch.Tensor | None = None,
    scaling: float | None = None,
    cost_aa: torch.Tensor | None = None,
    cost_bb: torch.Tensor | None = None,
) -> torch.Tensor:
    _check_op_cost(cost, "sinkhorn_divergence")
    return _sinkhorn_divergence(
        cost, eps=eps, n_iter=n_iter, a=a, b=b, scaling=scaling, cost_aa=cost_aa,
        cost_bb=cost_bb, mask=mask, check_cost=True,
    )


def _sinkhorn_divergence_fake(  # noqa: PLR0913
    cost: torch.Tensor,
    eps: float,
    n_iter: int,
    a: torch.Tensor,
    b: torch.Tensor,
    mask: torch.Tensor | None = None,
    scaling: float | None = None,
    cost_aa: torch.Tensor | None = None,
    cost_bb: torch.Tensor | None = None,
) -> torch.Tensor:
    del eps, n_iter, a, b, mask, scaling, cost_aa, cost_bb
    torch._check(cost.dim() == 3, lambda: "cost must be 3D (B, N, M)")
    return cost.new_empty(cost.size(0))


def _register(name: str, impl, fake) -> None:
    qualname = f"transport::{name}"
    if _has_op("transport", name):
        # the reference already defined the op (and its CPU path): add the
        # device kernel only
        torch.library.register_kernel(qualname, "cuda", impl)
        return
    op = torch.library.custom_op(qualname, impl, mutates_args=(), device_types="cuda")
    op.register_fake(fake)
    _LIBS.append(op)


_register("log_sinkhorn", _log_sinkhorn_impl, _log_sinkhorn_fake)
_register("unbalanced_sinkhorn", _unbalanced_sinkhorn_impl, _unbalanced_sinkhorn_fake)
_register("sinkhorn_divergence", _sinkhorn_divergence_impl, _sinkhorn_divergence_fake)
