"""Sinkhorn divergence on the gfx950 kernel.

The divergence is three potential-only kernel runs combined as the reference
does (transport/matrix/_sinkhorn_divergence.py:56-128).  The checks:

* against the same combination computed from the CPU oracle's potentials
  (oracle/sinkhorn.py), within 1e-5 of the largest of the three OT terms
  (the divergence is a difference of nearly equal terms, so its own relative
  error is not meaningful);
* the reference's own tests (test_transport_sinkhorn_divergence.py:9-61):
  scalar / per-batch shapes, symmetry under transposition, non-negativity
  when the self-costs share the geometry;
* the op entry with a mask and the solve() entry agree.
"""

from __future__ import annotations

import pytest
import torch

import torchmatch_amd  # noqa: F401
from oracle import sinkhorn as sk
import workloads
from torchmatch_amd.transport.matrix import Backend, solve

pytestmark = pytest.mark.gpu

TOL = 1e-5


def _oracle_divergence(cost, a, b, eps, n_iter, cost_aa=None, cost_bb=None):
    def ot(c, p, q):
        _, f, g, _, _ = sk.log_sinkhorn_plan(c, eps=eps, n_iter=n_iter, a=p, b=q)
        return (p * f).sum(-1) + (q * g).sum(-1)

    bsz, n, m = cost.shape
    c_aa = torch.zeros(bsz, n, n) if cost_aa is None else cost_aa.expand(bsz, n, n)
    c_bb = torch.zeros(bsz, m, m) if cost_bb is None else cost_bb.expand(bsz, m, m)
    ab, aa, bb = ot(cost, a, b), ot(c_aa, a, a), ot(c_bb, b, b)
    scale = torch.stack([ab.abs(), aa.abs(), bb.abs()]).amax(0)
    return -(ab - 0.5 * aa - 0.5 * bb), scale


@pytest.mark.parametrize(("B", "N", "M", "eps", "n_iter"), [
    (2, 40, 30, 0.1, 100),
    (1, 200, 300, 0.05, 150),
    (3, 64, 64, 0.5, 60),
])
def test_divergence_matches_oracle(B, N, M, eps, n_iter, device):
    cost = workloads.sinkhorn_points(B, N, M, 4, seed=N + M)
    a = workloads.dirichlet(B, N, 1.0, seed=3)
    b = workloads.dirichlet(B, M, 1.0, seed=4)
    want, scale = _oracle_divergence(cost, a, b, eps, n_iter)
    got = torch.ops.transport.sinkhorn_divergence(
        cost.to(device), eps, n_iter, a.to(device), b.to(device)
    ).cpu()
    err = ((got.double() - want.double()).abs() / scale.double()).max().item()
    print(f"divergence {(B, N, M, eps, n_iter)} err {err:.3e}", flush=True)
    assert err <= TOL


def test_divergence_with_self_costs_matches_oracle(device):
    g = torch.Generator().manual_seed(7)
    x = torch.randn(1, 50, 3, generator=g)
    y = torch.randn(1, 70, 3, generator=g)
    cost = torch.cdist(x, y).pow(2)
    c_xx = torch.cdist(x, x).pow(2)
    c_yy = torch.cdist(y, y).pow(2)
    a = torch.full((1, 50), 1 / 50)
    b = torch.full((1, 70), 1 / 70)
    want, scale = _oracle_divergence(cost, a, b, 0.2, 200, c_xx, c_yy)
    got = solve(cost[0].to(device), backend=Backend.SINKHORN_DIVERGENCE, reg=0.2,
                n_iter=200, cost_aa=c_xx[0].to(device), cost_bb=c_yy[0].to(device)).cpu()
    err = (abs(got.double().item() - want.double().item()) / scale.double().item())
    print(f"divergence with self costs err {err:.3e} value {got.item():.6f}", flush=True)
    assert err <= TOL
    assert got.item() >= -1e-5


def test_reference_shapes(device):
    # test_transport_sinkhorn_divergence.py:9-19
    out = solve(torch.rand(3, 4, dtype=torch.float64, device=device),
                backend=Backend.SINKHORN_DIVERGENCE, reg=0.1, n_iter=200)
    assert out.shape == () and torch.isfinite(out)
    out = solve(torch.rand(4, 3, 3, dtype=torch.float64, device=device),
                backend=Backend.SINKHORN_DIVERGENCE, reg=0.5, n_iter=200)
    assert out.shape == (4,)


def test_reference_symmetry(device):
    # test_transport_sinkhorn_divergence.py:22-40
    torch.manual_seed(0)
    cost_ab = torch.rand(3, 3, dtype=torch.float64)
    s_ab = solve(cost_ab.to(device), backend=Backend.SINKHORN_DIVERGENCE, reg=0.1, n_iter=300)
    s_ba = solve(cost_ab.T.contiguous().to(device), backend=Backend.SINKHORN_DIVERGENCE,
                 reg=0.1, n_iter=300)
    assert abs(s_ab.item() - s_ba.item()) < 1e-4


def test_reference_non_negative(device):
    # test_transport_sinkhorn_divergence.py:43-61
    torch.manual_seed(1)
    x = torch.rand(4, 3, dtype=torch.float64)
    y = torch.rand(4, 3, dtype=torch.float64)
    out = solve(torch.cdist(x, y).pow(2).to(device), backend=Backend.SINKHORN_DIVERGENCE,
                reg=0.5, n_iter=500, cost_aa=torch.cdist(x, x).pow(2).to(device),
                cost_bb=torch.cdist(y, y).pow(2).to(device))
    assert out.item() >= -1e-5


def test_mask_entry_matches_solve(device):
    cost = workloads.sinkhorn_points(2, 20, 25, 4, seed=5).to(device)
    mask = torch.rand(2, 20, 25, generator=torch.Generator().manual_seed(6)) > 0.2
    a = torch.full((2, 20), 1 / 20, device=device)
    b = torch.full((2, 25), 1 / 25, device=device)
    via_op = torch.ops.transport.sinkhorn_divergence(cost, 0.1, 80, a, b, mask=mask.to(device))
    via_solve = solve(cost, backend="sinkhorn_divergence", reg=0.1, n_iter=80, a=a, b=b,
                      mask=mask.to(device))
    assert torch.equal(via_op, via_solve)
