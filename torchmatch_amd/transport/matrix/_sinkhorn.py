"""Device log-domain Sinkhorn (balanced and unbalanced) behind the reference's ops.

Python surface mirrored from the reference:

* :func:`log_sinkhorn_plan`  -- ``transport/matrix/_log_sinkhorn.py:136-221``
* :func:`unbalanced_sinkhorn_plan` -- ``transport/matrix/_unbalanced_sinkhorn.py:30-103``
* :func:`sinkhorn_divergence` -- ``transport/matrix/_sinkhorn_divergence.py:56-128``
* ops ``transport::log_sinkhorn`` (``_log_sinkhorn.py:224-266``),
  ``transport::unbalanced_sinkhorn`` (``_unbalanced_sinkhorn.py:106-153``) and
  ``transport::sinkhorn_divergence`` (``_sinkhorn_divergence.py:131-173``),
  same schemas (inferred from the same Python signatures), same fakes.

The iteration itself runs in the gfx950 kernels of ``csrc/sinkhorn.hip`` via
``torch.ops.torchmatch_amd.sinkhorn``; this module only validates, builds the
epsilon schedule and shapes the results.  The kernels compute in float32
(float64 input is solved in float32 and the result cast back).  Device
tensors only: there is no host or torch-eager fallback.  Autograd through the
kernel is not provided (the reference's ``solve`` differentiates through
torch eager code instead).
"""

from __future__ import annotations

import torch

from torchmatch_amd._loader import _has_op
from torchmatch_amd._loader import load as _load
from torchmatch_amd.transport.matrix._schedule import build_eps_schedule
from torchmatch_amd.transport.matrix._validate import fuse_mask_into_cost, validate_cost

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


def _run(
    cost: torch.Tensor,
    a: torch.Tensor,
    b: torch.Tensor,
    schedule: list[float],
    rho: float,
    *,
    write_plan: bool = True,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    c32 = cost.to(torch.float32).contiguous()
    a32 = a.to(torch.float32).contiguous()
    b32 = b.to(torch.float32).contiguous()
    return torch.ops.torchmatch_amd.sinkhorn(c32, a32, b32, schedule, float(rho), write_plan)


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
    schedule = build_eps_schedule(cost=cost, reg=eps, n_iter=n_iter, scaling=scaling)
    b_size, rows, cols = cost.shape
    if b_size == 0:
        empty_plan = cost.new_empty(b_size, rows, cols)
        if return_potentials:
            return empty_plan, cost.new_empty(b_size, rows), cost.new_empty(b_size, cols)
        return empty_plan
    _require_device(cost, a, b, "log_sinkhorn")
    log_plan, log_u, log_v = _run(cost, a, b, schedule, 0.0)
    log_plan = log_plan.to(cost.dtype)
    if return_potentials:
        final_eps = schedule[-1]
        f = (-final_eps * log_u).to(cost.dtype)
        g = (-final_eps * log_v).to(cost.dtype)
        return log_plan, f, g
    return log_plan


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
        msg = (
            "torchmatch.transport.matrix.solve: rho must be positive for "
            f"UNBALANCED_SINKHORN, got {rho}"
        )
        raise ValueError(msg)
    schedule = build_eps_schedule(cost=cost, reg=eps, n_iter=n_iter, scaling=scaling)
    b_size, rows, cols = cost.shape
    if b_size == 0:
        return cost.new_empty(b_size, rows, cols)
    _require_device(cost, a, b, "unbalanced_sinkhorn")
    log_plan, _, _ = _run(cost, a, b, schedule, float(rho))
    return log_plan.to(cost.dtype)


def _potentials(cost, a, b, eps, n_iter, scaling):
    """(f, g) of ``log_sinkhorn_plan(..., return_potentials=True)`` without
    writing the plan (the divergence reads only the potentials)."""
    schedule = build_eps_schedule(cost=cost, reg=eps, n_iter=n_iter, scaling=scaling)
    b_size, rows, cols = cost.shape
    if b_size == 0:
        return cost.new_empty(b_size, rows), cost.new_empty(b_size, cols)
    _require_device(cost, a, b, "sinkhorn_divergence")
    _, log_u, log_v = _run(cost, a, b, schedule, 0.0, write_plan=False)
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
    batch = cost.size(0)
    n = a.size(-1)
    m = b.size(-1)

    def ot(c, p, q):
        f, g = _potentials(c, p, q, eps, n_iter, scaling)
        return (p * f).sum(dim=-1) + (q * g).sum(dim=-1)

    ot_ab = ot(cost, a, b)
    ot_aa = ot(_expand_self_cost(cost_aa, cost, batch, n), a, a)
    ot_bb = ot(_expand_self_cost(cost_bb, cost, batch, m), b, b)
    return -(ot_ab - 0.5 * ot_aa - 0.5 * ot_bb)


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
    validate_cost(cost)
    if cost.ndim != 3:
        msg = (
            "torch.ops.transport.log_sinkhorn: cost.ndim must be 3, got "
            f"{cost.ndim}. Call torchmatch.transport.matrix.solve(...) for "
            "2-D ergonomic dispatch."
        )
        raise ValueError(msg)
    cost = fuse_mask_into_cost(cost, mask)
    return log_sinkhorn_plan(cost, eps=eps, n_iter=n_iter, a=a, b=b, scaling=scaling)


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
    validate_cost(cost)
    if cost.ndim != 3:
        msg = (
            "torch.ops.transport.unbalanced_sinkhorn: cost.ndim must be 3, "
            f"got {cost.ndim}"
        )
        raise ValueError(msg)
    if rho <= 0:
        msg = "torch.ops.transport.unbalanced_sinkhorn: rho must be positive"
        raise ValueError(msg)
    cost = fuse_mask_into_cost(cost, mask)
    return unbalanced_sinkhorn_plan(
        cost, eps=eps, n_iter=n_iter, rho=rho, a=a, b=b, scaling=scaling
    )


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
    validate_cost(cost)
    if cost.ndim != 3:
        msg = (
            "torch.ops.transport.sinkhorn_divergence: cost.ndim must be 3, "
            f"got {cost.ndim}"
        )
        raise ValueError(msg)
    cost = fuse_mask_into_cost(cost, mask)
    return sinkhorn_divergence(
        cost, eps=eps, n_iter=n_iter, a=a, b=b, scaling=scaling,
        cost_aa=cost_aa, cost_bb=cost_bb,
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
