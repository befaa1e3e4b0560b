"""float64 Sinkhorn: the reference iterates in the cost's dtype
(transport/matrix/_log_sinkhorn.py:184,191; _unbalanced_sinkhorn.py:60,67), so
float64 costs run the float64 kernels (csrc/sinkhorn64.hip).

Held against the CPU oracle in float64: max |log P - log P_ref| over finite
entries and max-abs of f / g within 1e-9 (both sides are float64; they differ
only in summation order, ~1e-15 per operation, accumulated over the
iterations), identical -inf patterns, float64 outputs.
"""

from __future__ import annotations

import pytest
import torch

import sk_parity
import torchmatch_amd  # noqa: F401
from oracle import sinkhorn as sk
import workloads
from torchmatch_amd.transport.matrix import solve

pytestmark = pytest.mark.gpu

TOL64 = 1e-9


def _cost64(B, N, M, seed):
    return workloads.sinkhorn_points(B, N, M, 8, seed=seed).double()


@pytest.mark.parametrize(("B", "N", "M", "eps", "n_iter"), [
    (2, 64, 80, 0.1, 60), (1, 300, 200, 0.05, 100), (3, 17, 1000, 0.05, 40),
])
def test_log_sinkhorn_f64_matches_oracle(B, N, M, eps, n_iter, device):
    cost = _cost64(B, N, M, seed=N + M)
    cost[0, 3, :] = float("inf")          # all-+inf row
    cost[B - 1, :, 5] = float("inf")      # all-+inf column
    cost[0, 7, M // 4: M // 2] = float("inf")
    a = workloads.dirichlet(B, N, 1.0, seed=1).double()
    b = workloads.dirichlet(B, M, 1.0, seed=2).double()
    ref_plan, ref_f, ref_g, _, _ = sk.log_sinkhorn_plan(cost, eps=eps, n_iter=n_iter, a=a, b=b)
    plan, f, g = solve(cost.to(device), reg=eps, n_iter=n_iter, a=a.to(device), b=b.to(device),
                       unpack=True)
    assert plan.dtype == f.dtype == g.dtype == torch.float64
    ep, ef, eg = (sk_parity.logp_err(plan, ref_plan), sk_parity.pot_err(f, ref_f),
                  sk_parity.pot_err(g, ref_g))
    print(f"f64 log_sinkhorn {(B, N, M)}: plan {ep:.2e} f {ef:.2e} g {eg:.2e}", flush=True)
    assert ep <= TOL64 and ef <= TOL64 and eg <= TOL64


def test_unbalanced_f64_matches_oracle(device):
    B, N, M = 2, 120, 90
    cost = _cost64(B, N, M, seed=5)
    a = workloads.dirichlet(B, N, 1.0, seed=3).double()
    b = workloads.dirichlet(B, M, 1.3, seed=4).double()
    ref = sk.unbalanced_sinkhorn_plan(cost, eps=0.02, n_iter=80, rho=1.0, a=a, b=b)[0]
    plan = torch.ops.transport.unbalanced_sinkhorn(cost.to(device), 0.02, 80, 1.0, a.to(device),
                                                   b.to(device))
    assert plan.dtype == torch.float64
    ep = sk_parity.logp_err(plan, ref)
    print(f"f64 unbalanced: plan {ep:.2e}", flush=True)
    assert ep <= TOL64


def test_f64_scaling_and_mask(device):
    cost = _cost64(1, 90, 70, seed=8)
    a = workloads.uniform_marginal(1, 90).double()
    b = workloads.uniform_marginal(1, 70).double()
    ref = sk.log_sinkhorn_plan(cost, eps=0.05, n_iter=50, a=a, b=b, scaling=0.6)[0]
    plan = solve(cost.to(device), reg=0.05, n_iter=50, a=a.to(device), b=b.to(device),
                 scaling=0.6)
    assert sk_parity.logp_err(plan, ref) <= TOL64
    mask = torch.rand(1, 90, 70, generator=torch.Generator().manual_seed(2)) > 0.3
    ref = sk.log_sinkhorn_plan(cost.masked_fill(~mask, float("inf")), eps=0.05, n_iter=50,
                               a=a, b=b)[0]
    plan = torch.ops.transport.log_sinkhorn(cost.to(device), 0.05, 50, a.to(device),
                                            b.to(device), mask.to(device))
    assert plan.dtype == torch.float64
    assert sk_parity.logp_err(plan, ref) <= TOL64


def test_f64_is_not_float32(device):
    """The float64 path does not round through float32: its plan differs from
    the float32 solve of the same cost by float32-size amounts, while it
    agrees with the float64 oracle to ~1e-12."""
    cost = _cost64(1, 64, 64, seed=11)
    p64 = solve(cost.to(device), reg=0.05, n_iter=40)
    p32 = solve(cost.float().to(device), reg=0.05, n_iter=40)
    ref = sk.log_sinkhorn_plan(cost, eps=0.05, n_iter=40, a=workloads.uniform_marginal(1, 64)
                               .double(), b=workloads.uniform_marginal(1, 64).double())[0]
    assert sk_parity.logp_err(p64, ref) <= TOL64
    assert (p64.cpu() - p32.double().cpu()).abs().max().item() > 1e-8


def test_batch_above_grid_limit_f64(device):
    """70,000 problems (more than one 65,535-block grid dimension holds): the
    column kernel strides over (batch, strip) pairs."""
    B, N, M = 70_000, 2, 3
    cost = torch.rand(B, N, M, generator=torch.Generator().manual_seed(21), dtype=torch.float64)
    a = torch.full((B, N), 1.0 / N, dtype=torch.float64)
    b = torch.full((B, M), 1.0 / M, dtype=torch.float64)
    ref = sk.log_sinkhorn_plan(cost, eps=0.1, n_iter=12, a=a, b=b)[0]
    plan = torch.ops.transport.log_sinkhorn(cost.to(device), 0.1, 12, a.to(device), b.to(device))
    ep = sk_parity.logp_err(plan, ref)
    print(f"f64 B={B}: plan {ep:.2e}", flush=True)
    assert ep <= TOL64
