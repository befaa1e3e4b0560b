"""Pins the Sinkhorn oracle (oracle/sinkhorn.py) and the shared schedule.

The reference computes Sinkhorn with torch calls; the oracle repeats them.
Its values are pinned here by things that do not depend on re-typing the
same formula:

* an independent float64 implementation written against numpy/scipy
  (``scipy.special.logsumexp``) of the recurrence in
  transport/matrix/_log_sinkhorn.py:194-215 / _unbalanced_sinkhorn.py:70-103;
* closed forms from the reference tests (1x1 unbalanced,
  test_transport_unbalanced_sinkhorn.py:59-87; uniform cost,
  test_transport_log_sinkhorn.py:12-21);
* invariants: marginals after convergence, -inf patterns, batch decoupling;
* a planted mistake (swapped half-steps) that the independent check rejects.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
from scipy.special import logsumexp

from oracle import sinkhorn as sk
from torchmatch_amd.transport.matrix._schedule import build_eps_schedule


def numpy_sinkhorn(cost, a, b, eps_list, rho=None, swap_halves=False):
    """Independent float64 restatement (numpy + scipy), per batch element."""
    cost = np.asarray(cost, np.float64)
    out = []
    for c, ai, bi in zip(cost, np.asarray(a, np.float64), np.asarray(b, np.float64)):
        n, m = c.shape
        row_inf = np.all(np.isinf(c), axis=1)
        col_inf = np.all(np.isinf(c), axis=0)
        with np.errstate(divide="ignore"):
            lmu, lnu = np.log(ai), np.log(bi)
        lu, lv = np.zeros(n), np.zeros(m)

        def upd_u(lk, lv, lu, damp):
            lse = logsumexp(lk + lv[None, :], axis=1)
            lse[row_inf] = -np.inf
            new = damp * (lmu - lse)
            return np.where(np.isfinite(lse), new, lu)

        def upd_v(lk, lu, lv, damp):
            lse = logsumexp(lk + lu[:, None], axis=0)
            lse[col_inf] = -np.inf
            new = damp * (lnu - lse)
            return np.where(np.isfinite(lse), new, lv)

        for e in eps_list:
            damp = 1.0 if rho is None else 1.0 / (1.0 + e / rho)
            with np.errstate(invalid="ignore"):
                lk = -c / e
            if swap_halves:
                lv = upd_v(lk, lu, lv, damp)
                lu = upd_u(lk, lv, lu, damp)
            else:
                lu = upd_u(lk, lv, lu, damp)
                lv = upd_v(lk, lu, lv, damp)
        out.append(lu[:, None] + (-c / eps_list[-1]) + lv[None, :])
    return np.stack(out)


def _problem(seed, b=2, n=7, m=5, inf_frac=0.0):
    g = torch.Generator().manual_seed(seed)
    c = torch.rand(b, n, m, dtype=torch.float64, generator=g) * 2
    if inf_frac:
        c[torch.rand(b, n, m, generator=g) < inf_frac] = float("inf")
    a = torch.rand(b, n, dtype=torch.float64, generator=g) + 0.1
    bb = torch.rand(b, m, dtype=torch.float64, generator=g) + 0.1
    return c, a / a.sum(1, keepdim=True), bb / bb.sum(1, keepdim=True)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_balanced_matches_independent_float64(seed):
    c, a, b = _problem(seed, inf_frac=0.15 if seed == 2 else 0.0)
    ref = numpy_sinkhorn(c, a, b, [0.2] * 40)
    got = sk.log_sinkhorn_plan(c, eps=0.2, n_iter=40, a=a, b=b)[0].numpy()
    assert np.array_equal(np.isneginf(got), np.isneginf(ref))
    fin = np.isfinite(ref)
    np.testing.assert_allclose(got[fin], ref[fin], rtol=0, atol=1e-12)


def test_unbalanced_matches_independent_float64():
    c, a, b = _problem(4)
    ref = numpy_sinkhorn(c, a, b * 1.3, [0.1] * 60, rho=0.7)
    got = sk.unbalanced_sinkhorn_plan(c, eps=0.1, n_iter=60, rho=0.7, a=a, b=b * 1.3)[0]
    np.testing.assert_allclose(got.numpy(), ref, rtol=0, atol=1e-12)


def test_eps_scaling_matches_independent_float64():
    c, a, b = _problem(5)
    sched = build_eps_schedule(cost=c, reg=0.05, n_iter=30, scaling=0.6)
    ref = numpy_sinkhorn(c, a, b, sched)
    got = sk.log_sinkhorn_plan(c, eps=0.05, n_iter=30, a=a, b=b, scaling=0.6)[0].numpy()
    np.testing.assert_allclose(got, ref, rtol=0, atol=1e-11)


def test_planted_mistake_is_caught():
    """Swapping the two half-steps changes the result beyond the tolerance."""
    c, a, b = _problem(6)
    wrong = numpy_sinkhorn(c, a, b, [0.2] * 5, swap_halves=True)
    got = sk.log_sinkhorn_plan(c, eps=0.2, n_iter=5, a=a, b=b)[0].numpy()
    assert np.abs(got - wrong).max() > 1e-6


def test_unbalanced_1x1_closed_form():
    a0, b0, c00, rho, eps = 0.7, 0.9, 0.3, 0.5, 0.1
    expected = (rho * (math.log(a0) + math.log(b0)) - c00) / (eps + 2.0 * rho)
    got = sk.unbalanced_sinkhorn_plan(
        torch.tensor([[[c00]]], dtype=torch.float64), eps=eps, n_iter=2000, rho=rho,
        a=torch.tensor([[a0]], dtype=torch.float64), b=torch.tensor([[b0]], dtype=torch.float64),
    )[0]
    assert abs(got.item() - expected) < 1e-10


def test_uniform_cost_uniform_plan():
    c = torch.ones(1, 4, 4, dtype=torch.float64)
    a = torch.full((1, 4), 0.25, dtype=torch.float64)
    plan = sk.log_sinkhorn_plan(c, eps=0.1, n_iter=100, a=a, b=a)[0].exp()
    assert torch.allclose(plan, torch.full_like(plan, 1 / 16), atol=1e-12)


def test_marginals_converge_and_forbidden_rows():
    c, a, b = _problem(7, n=6, m=6)
    c[0, 2, :] = float("inf")
    a[0, 2] = 0.0
    a = a / a.sum(1, keepdim=True)
    plan = sk.log_sinkhorn_plan(c, eps=0.3, n_iter=500, a=a, b=b)[0]
    assert torch.isneginf(plan[0, 2]).all()
    assert not torch.isnan(plan).any()
    p = plan.exp()
    assert torch.allclose(p.sum(2), a, atol=1e-8)
    assert torch.allclose(p.sum(1), b, atol=1e-8)


def test_batch_decouples():
    c, a, b = _problem(8, b=3)
    whole = sk.log_sinkhorn_plan(c, eps=0.2, n_iter=30, a=a, b=b)[0]
    for i in range(3):
        one = sk.log_sinkhorn_plan(c[i:i + 1], eps=0.2, n_iter=30, a=a[i:i + 1], b=b[i:i + 1])[0]
        assert torch.equal(one[0], whole[i])


# ---- schedule (transport/matrix/_schedule.py:21-76; test_transport_schedule.py) ----

def test_schedule_flat_and_geometric():
    c = torch.tensor([[0.0, 4.0], [1.0, float("inf")]])
    assert build_eps_schedule(cost=c, reg=0.1, n_iter=3, scaling=None) == [0.1, 0.1, 0.1]
    s = build_eps_schedule(cost=c, reg=0.1, n_iter=6, scaling=0.5)
    assert s[0] == 2.0 and s[1] == 1.0 and s[-1] == 0.1
    assert all(x >= 0.1 for x in s)
    assert s == sk.eps_schedule(c, 0.1, 6, 0.5)


@pytest.mark.parametrize(("kw", "msg"), [
    ({"reg": 0.0, "n_iter": 3, "scaling": None}, "reg must be positive"),
    ({"reg": 0.1, "n_iter": 0, "scaling": None}, "n_iter must be >= 1"),
    ({"reg": 0.1, "n_iter": 3, "scaling": 1.0}, "scaling must be in"),
])
def test_schedule_errors(kw, msg):
    with pytest.raises(ValueError, match=msg):
        build_eps_schedule(cost=torch.ones(2, 2), **kw)


# ---- the order of the two half-steps, fixed by the mathematics ---------------
# (_log_sinkhorn.py:194-215: the row half-step first, with the previous log_v,
# then the column half-step with the new log_u)


def _small_problem(seed, B=2, N=7, M=5):
    g = torch.Generator().manual_seed(seed)
    cost = torch.rand(B, N, M, generator=g, dtype=torch.float64) * 3
    a = torch.rand(B, N, generator=g, dtype=torch.float64) + 0.1
    b = torch.rand(B, M, generator=g, dtype=torch.float64) + 0.1
    b = b / b.sum(-1, keepdim=True) * a.sum(-1, keepdim=True)   # balanced masses
    return cost, a, b


@pytest.mark.parametrize("seed", [0, 1])
def test_one_iteration_closed_form(seed):
    """n_iter = 1 from log_u = log_v = 0: log_u = log a - LSE_j(-C/eps), then
    log_v = log b - LSE_i(-C/eps + log_u), written out with plain exp/log
    sums per entry.  Swapping the half-steps, dropping log_u from the column
    update or using the row update's old log_v all change the result."""
    cost, a, b = _small_problem(seed)
    eps = 0.3
    _, _, _, lu, lv = sk.log_sinkhorn_plan(cost, eps=eps, n_iter=1, a=a, b=b)
    B, N, M = cost.shape
    for k in range(B):
        c = cost[k].numpy()
        for i in range(N):
            want = math.log(a[k, i].item()) - math.log(sum(math.exp(-c[i, j] / eps)
                                                            for j in range(M)))
            assert abs(lu[k, i].item() - want) < 1e-12
        for j in range(M):
            s = sum(math.exp(-c[i, j] / eps + lu[k, i].item()) for i in range(N))
            want = math.log(b[k, j].item()) - math.log(s)
            assert abs(lv[k, j].item() - want) < 1e-12


def test_one_iteration_unbalanced_closed_form():
    """Same, with the damping 1 / (1 + eps / rho) of _unbalanced_sinkhorn.py:71
    applied to each half-step's update."""
    cost, a, b = _small_problem(3)
    eps, rho = 0.3, 0.8
    damp = 1.0 / (1.0 + eps / rho)
    _, lu, lv = sk.unbalanced_sinkhorn_plan(cost, eps=eps, n_iter=1, rho=rho, a=a, b=b)
    B, N, M = cost.shape
    for k in range(B):
        c = cost[k].numpy()
        for i in range(N):
            lse = math.log(sum(math.exp(-c[i, j] / eps) for j in range(M)))
            assert abs(lu[k, i].item() - damp * (math.log(a[k, i].item()) - lse)) < 1e-12
        for j in range(M):
            lse = math.log(sum(math.exp(-c[i, j] / eps + lu[k, i].item()) for i in range(N)))
            assert abs(lv[k, j].item() - damp * (math.log(b[k, j].item()) - lse)) < 1e-12


@pytest.mark.parametrize("n_iter", [1, 2, 3, 7])
def test_column_marginals_exact_after_any_iteration(n_iter):
    """The balanced step ends with the column half-step, so after ANY number
    of iterations the plan's column sums equal b (to float64 rounding) while
    the row sums do not yet equal a (far from converged at these n_iter).
    A restatement with the half-steps swapped has it the other way round."""
    cost, a, b = _small_problem(5, B=2, N=9, M=6)
    eps = 0.2
    plan = sk.log_sinkhorn_plan(cost, eps=eps, n_iter=n_iter, a=a, b=b)[0].exp()
    col_err = (plan.sum(1) - b).abs().max().item()
    row_err = (plan.sum(2) - a).abs().max().item()
    assert col_err < 1e-12
    assert row_err > 1e-6
    lp = numpy_sinkhorn(cost.numpy(), a.numpy(), b.numpy(), [eps] * n_iter,
                        swap_halves=True)
    swapped = np.exp(lp)
    assert np.abs(swapped.sum(2) - a.numpy()).max() < 1e-12      # rows exact instead
    assert np.abs(swapped.sum(1) - b.numpy()).max() > 1e-6
