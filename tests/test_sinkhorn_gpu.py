"""Parity of the gfx950 Sinkhorn kernels with the reference computation.

The oracle (oracle/sinkhorn.py) is the reference's torch code restated op for
op on CPU.  Every parity case runs it twice, in float32 (the reference's own
arithmetic) and in float64, and holds the kernels to element-wise measures
(tests/sk_parity.py): max |log P - log P_ref| over the finite plan entries
(the relative error of each plan entry) and the max-abs error of the
potentials f = -eps log_u, g = -eps log_v, each within
max(1e-5, 2.5 x the float32 oracle's own drift from float64); the -inf pattern
of the log plan must be identical.  Full-size C4 and C5 are in
tests/test_sinkhorn_fullsize_gpu.py.
"""

from __future__ import annotations

import math

import pytest
import torch

import torchmatch_amd  # noqa: F401
from oracle import sinkhorn as sk
import sk_parity
import workloads
from torchmatch_amd.transport.matrix import Backend, marginal_error, solve

pytestmark = pytest.mark.gpu


def _balanced_refs(cost, eps, n_iter, a, b, scaling=None):
    r32 = sk.log_sinkhorn_plan(cost, eps=eps, n_iter=n_iter, a=a, b=b, scaling=scaling)
    r64 = sk.log_sinkhorn_plan(cost, eps=eps, n_iter=n_iter, a=a, b=b, scaling=scaling,
                               dtype=torch.float64)
    return ({"plan": r32[0], "f": r32[1], "g": r32[2]},
            {"plan": r64[0], "f": r64[1], "g": r64[2]})


def _unbalanced_refs(cost, eps, n_iter, rho, a, b):
    r32 = sk.unbalanced_sinkhorn_plan(cost, eps=eps, n_iter=n_iter, rho=rho, a=a, b=b)
    r64 = sk.unbalanced_sinkhorn_plan(cost, eps=eps, n_iter=n_iter, rho=rho, a=a, b=b,
                                      dtype=torch.float64)
    return {"plan": r32[0]}, {"plan": r64[0]}


def _check_balanced(label, cost, eps, n_iter, a, b, device, scaling=None, mask=None):
    """solve(unpack=True) on the device vs the oracle at both precisions."""
    c_ref = cost if mask is None else cost.masked_fill(~mask, float("inf"))
    r32, r64 = _balanced_refs(c_ref, eps, n_iter, a, b, scaling)
    if mask is None:
        plan, f, g = solve(cost.to(device), reg=eps, n_iter=n_iter, a=a.to(device),
                           b=b.to(device), scaling=scaling, unpack=True)
        got = {"plan": plan, "f": f, "g": g}
    else:
        plan = torch.ops.transport.log_sinkhorn(cost.to(device), eps, n_iter, a.to(device),
                                                b.to(device), mask.to(device), scaling)
        got = {"plan": plan}
    torch.cuda.synchronize()
    return sk_parity.check(label, got, r32, r64)


def _check_unbalanced(label, cost, eps, n_iter, rho, a, b, device):
    r32, r64 = _unbalanced_refs(cost, eps, n_iter, rho, a, b)
    plan = torch.ops.transport.unbalanced_sinkhorn(cost.to(device), eps, n_iter, rho,
                                                   a.to(device), b.to(device))
    torch.cuda.synchronize()
    return sk_parity.check(label, {"plan": plan}, r32, r64)


CASES = [
    # B, N, M, eps, n_iter
    (2, 64, 64, 0.1, 50),
    (2, 256, 256, 0.05, 200),
    (3, 300, 200, 0.1, 100),
    (1, 130, 517, 0.05, 80),
    (2, 1024, 1024, 0.05, 60),
    (3, 77, 1028, 0.05, 60),
    (2, 200, 2048, 0.05, 60),
    # rows longer than one 2048-column chunk: several waves per row
    (1, 100, 3000, 0.05, 40),
    (1, 48, 4100, 0.05, 40),
    (1, 32, 16384, 0.05, 30),
    (1, 16, 40000, 0.1, 20),
    # fewer rows than a block's row groups / waves
    (1, 1, 256, 0.05, 20),
    (2, 3, 1024, 0.05, 20),
    (1, 2, 9000, 0.05, 20),
]


@pytest.mark.parametrize(("B", "N", "M", "eps", "n_iter"), CASES)
def test_log_sinkhorn_matches_oracle(B, N, M, eps, n_iter, device):
    cost = workloads.sinkhorn_points(B, N, M, 8, seed=N + M)
    a = workloads.dirichlet(B, N, 1.0, seed=1)
    b = workloads.dirichlet(B, M, 1.0, seed=2)
    print(f"log_sinkhorn case {(B, N, M, eps, n_iter)}", flush=True)
    _check_balanced("log_sinkhorn", cost, eps, n_iter, a, b, device)


@pytest.mark.parametrize(("B", "N", "M", "eps", "n_iter", "rho"), [
    (2, 64, 80, 0.1, 60, 1.0),
    (1, 500, 300, 0.02, 100, 1.0),
    (2, 256, 256, 0.05, 100, 0.5),
    (1, 64, 8192, 0.02, 50, 1.0),
])
def test_unbalanced_matches_oracle(B, N, M, eps, n_iter, rho, device):
    cost = workloads.sinkhorn_points(B, N, M, 8, seed=3)
    a = workloads.dirichlet(B, N, 1.0, seed=4)
    b = workloads.dirichlet(B, M, 1.3, seed=5)
    print(f"unbalanced case {(B, N, M, eps, n_iter, rho)}", flush=True)
    _check_unbalanced("unbalanced", cost, eps, n_iter, rho, a, b, device)


# The step's two kernel shapes: one pass over K per step (row LSE, then the
# same rows folded into per-column partials) and the two-sweep step ("0"); the
# long-row pass in its 8-wave shape too.  Each is held to the oracle.
STEP_SHAPES = [
    # env value, (B, N, M); each case also holds all-+inf rows and columns
    (None, (2, 150, 1500)),
    ("0", (2, 150, 1500)),
    (None, (1, 40, 12000)),
    ("8x1x8", (1, 40, 12000)),
    ("0", (1, 40, 12000)),
]


@pytest.mark.parametrize(("env", "shape"), STEP_SHAPES)
def test_step_shapes_match_oracle(env, shape, device, monkeypatch):
    if env is None:
        monkeypatch.delenv("TORCHMATCH_AMD_SINKHORN_FUSED", raising=False)
    else:
        monkeypatch.setenv("TORCHMATCH_AMD_SINKHORN_FUSED", env)
    B, N, M = shape
    cost = workloads.sinkhorn_points(B, N, M, 8, seed=N + 7)
    cost[0, 3, :] = float("inf")           # all-+inf row
    cost[B - 1, :, 5] = float("inf")       # all-+inf column
    cost[0, 9, M // 3: M // 2] = float("inf")
    a = workloads.dirichlet(B, N, 1.0, seed=21)
    b = workloads.dirichlet(B, M, 1.0, seed=22)
    print(f"step shape env={env} {shape}", flush=True)
    _check_balanced("balanced", cost, 0.05, 40, a, b, device)
    _check_unbalanced("unbalanced", cost, 0.05, 40, 0.7, a, b * 1.3, device)


# Row chunks per batch of the one-read step: more than 64 chunks take the
# 16-wave column merge (C5 has 256).  (1, 600, 4100): 75 chunks of the 4-wave
# long-row shape; (1, 1024, 9000): 128 chunks of the 16-wave shape.  Each runs
# with the default shift window (merged sums) and with the window closed, so
# that every column after the first step takes the 16-wave exact recompute.
@pytest.mark.parametrize("window", [None, "0"])
@pytest.mark.parametrize(("N", "M"), [(600, 4100), (1024, 9000)])
def test_many_chunk_merge_matches_oracle(N, M, window, device, monkeypatch):
    if window is None:
        monkeypatch.delenv("TORCHMATCH_AMD_SINKHORN_SHIFT_WINDOW", raising=False)
    else:
        monkeypatch.setenv("TORCHMATCH_AMD_SINKHORN_SHIFT_WINDOW", window)
    cost = workloads.sinkhorn_points(1, N, M, 8, seed=N + M + 1)
    cost[0, 7, :] = float("inf")
    cost[0, :, 11] = float("inf")
    a = workloads.dirichlet(1, N, 1.0, seed=41)
    b = workloads.dirichlet(1, M, 1.0, seed=42)
    print(f"many-chunk merge {(1, N, M)} window={window}", flush=True)
    _check_balanced("balanced", cost, 0.05, 30, a, b, device)
    _check_unbalanced("unbalanced", cost, 0.02, 30, 1.0, a, b * 1.3, device)


@pytest.mark.parametrize(("B", "N", "M"), [(2, 300, 1024), (1, 64, 9000)])
def test_exact_column_recompute_matches_oracle(B, N, M, device, monkeypatch):
    """The fused step sums each column against the previous step's column LSE
    and recomputes exactly from the cost any column whose shifted total falls
    outside the accepted window.  Natural inputs rarely leave a 16-bit window
    (the column LSE moves ~3 per step), so the window is closed here and every
    column of every step after the first takes the recompute."""
    monkeypatch.setenv("TORCHMATCH_AMD_SINKHORN_SHIFT_WINDOW", "0")
    cost = workloads.sinkhorn_points(B, N, M, 8, seed=N + 3)
    cost[0, 2, :] = float("inf")
    cost[0, :, 9] = float("inf")
    a = workloads.dirichlet(B, N, 1.0, seed=5)
    b = workloads.dirichlet(B, M, 1.0, seed=6)
    print(f"exact recompute {(B, N, M)}", flush=True)
    _check_balanced("recompute", cost, 0.05, 25, a, b, device)


def test_forbidden_cells_rows_and_columns(device):
    cost = workloads.sinkhorn_points(2, 40, 30, 4, seed=9)
    cost[0, 3, :] = float("inf")         # all-+inf row
    cost[1, :, 7] = float("inf")         # all-+inf column
    cost[0, 5, 2] = float("inf")
    cost[1, 9, 11] = float("inf")
    a = workloads.uniform_marginal(2, 40)
    b = workloads.uniform_marginal(2, 30)
    plan, f, g = solve(cost.to(device), reg=0.1, n_iter=100, a=a.to(device), b=b.to(device),
                       unpack=True)
    assert torch.isneginf(plan[0, 3]).all() and torch.isneginf(plan[1, :, 7]).all()
    assert not torch.isnan(plan).any()
    _check_balanced("forbidden", cost, 0.1, 100, a, b, device)


def test_forbidden_rows_long_rows(device):
    """All-+inf rows and columns with rows split over several waves."""
    cost = workloads.sinkhorn_points(1, 24, 6000, 4, seed=11)
    cost[0, 5, :] = float("inf")
    cost[0, :, 4321] = float("inf")
    cost[0, 7, 2000:4500] = float("inf")
    a = workloads.dirichlet(1, 24, 1.0, seed=12)
    b = workloads.dirichlet(1, 6000, 1.0, seed=13)
    print("forbidden long rows", flush=True)
    _check_balanced("forbidden long rows", cost, 0.1, 30, a, b, device)


def test_mask_argument_and_op_entry(device):
    cost = workloads.sinkhorn_points(2, 50, 60, 8, seed=10)
    mask = torch.rand(2, 50, 60, generator=torch.Generator().manual_seed(0)) > 0.2
    a = workloads.uniform_marginal(2, 50)
    b = workloads.uniform_marginal(2, 60)
    _check_balanced("mask op", cost, 0.1, 70, a, b, device, mask=mask)


def test_eps_scaling_schedule(device):
    cost = workloads.sinkhorn_points(1, 120, 90, 8, seed=12)
    a = workloads.uniform_marginal(1, 120)
    b = workloads.uniform_marginal(1, 90)
    r32, r64 = _balanced_refs(cost, 0.05, 120, a, b, scaling=0.7)
    plan = solve(cost[0].to(device), reg=0.05, n_iter=120, scaling=0.7)
    sk_parity.check("scaling 2-D", {"plan": plan.unsqueeze(0)}, r32, r64)


@pytest.mark.parametrize(("N", "M"), [(200, 1500), (40, 9000)])
def test_eps_scaling_and_mask_on_fused_step(N, M, device):
    """epsilon scaling on shapes that take the one-read step: K is rebuilt
    while epsilon decays (each such step folds exactly), then the shifted
    column sums resume once epsilon settles at reg; and a keep mask."""
    cost = workloads.sinkhorn_points(1, N, M, 8, seed=M)
    a = workloads.dirichlet(1, N, 1.0, seed=7)
    b = workloads.dirichlet(1, M, 1.0, seed=8)
    print(f"scaling / mask {(N, M)}", flush=True)
    _check_balanced("scaling", cost, 0.05, 30, a, b, device, scaling=0.5)
    mask = torch.rand(1, N, M, generator=torch.Generator().manual_seed(1)) > 0.3
    _check_balanced("mask", cost, 0.05, 30, a, b, device, mask=mask)


@pytest.mark.parametrize("groups", ["1", "2", "3", "4"])
def test_batch_groups_match_oracle(groups, device, monkeypatch):
    """The fused step runs batch groups on separate streams (two by default).
    Every group count, including uneven splits of B = 5, gives the oracle's
    plan under epsilon scaling (K rebuilt between segments of steps), and the
    same bits as one group: each batch's arithmetic does not depend on the
    split."""
    B, N, M = 5, 120, 1028
    cost = workloads.sinkhorn_points(B, N, M, 8, seed=31)
    cost[2, 4, :] = float("inf")
    a = workloads.dirichlet(B, N, 1.0, seed=32)
    b = workloads.dirichlet(B, M, 1.0, seed=33)
    r32, r64 = _balanced_refs(cost, 0.05, 30, a, b, scaling=0.5)
    args = (cost.to(device),)
    kw = dict(reg=0.05, n_iter=30, a=a.to(device), b=b.to(device), scaling=0.5)
    monkeypatch.setenv("TORCHMATCH_AMD_SINKHORN_GROUPS", groups)
    plan = solve(*args, **kw)
    monkeypatch.setenv("TORCHMATCH_AMD_SINKHORN_GROUPS", "1")
    one = solve(*args, **kw)
    torch.cuda.synchronize()
    sk_parity.check(f"groups {groups}", {"plan": plan}, r32, r64)
    assert torch.equal(plan, one)


def test_uniform_cost_gives_uniform_plan(device):
    """test_transport_log_sinkhorn.py:12-21 (closed form)."""
    cost = torch.ones(4, 4, device=device)
    plan = solve(cost, reg=0.1, n_iter=100).exp()
    assert torch.allclose(plan, torch.full_like(plan, 1 / 16), atol=1e-6)


def test_unbalanced_1x1_closed_form(device):
    """test_transport_unbalanced_sinkhorn.py:59-87, at float32 precision."""
    a0, b0, c00, rho, eps = 0.7, 0.9, 0.3, 0.5, 0.1
    expected = (rho * (math.log(a0) + math.log(b0)) - c00) / (eps + 2.0 * rho)
    log_plan = solve(
        torch.tensor([[[c00]]], device=device), backend=Backend.UNBALANCED_SINKHORN,
        reg=eps, n_iter=2000, rho=rho,
        a=torch.tensor([[a0]], device=device), b=torch.tensor([[b0]], device=device),
    )
    assert abs(log_plan.item() - expected) < 1e-6


def test_c4_shape_converges(device):
    """C4 at full size (16, 2048, 2048), eps 0.05, 200 iterations: marginals."""
    cost = workloads.sinkhorn_points(16, 2048, 2048, 8, seed=0).to(device)
    a = torch.full((16, 2048), 1 / 2048, device=device)
    plan = solve(cost, reg=0.05, n_iter=200, a=a, b=a)
    row_err, col_err = marginal_error(plan, a, a)
    print(f"C4 marginal error rows {row_err:.3e} cols {col_err:.3e}", flush=True)
    assert col_err < 1e-6          # the last half-step fixes the columns
    assert row_err < 1e-6
    assert not torch.isnan(plan).any()


def test_potentials_reconstruct_plan(device):
    """log_plan = (-f - C - g) / eps (balanced, by construction of the plan)."""
    cost = workloads.sinkhorn_points(2, 300, 400, 8, seed=13)
    plan, f, g = solve(cost.to(device), reg=0.1, n_iter=50, unpack=True)
    rec = (-f[:, :, None] - cost.to(device) - g[:, None, :]) / 0.1
    assert (rec - plan).abs().max().item() < 1e-3


def test_cpu_tensor_rejected():
    with pytest.raises(ValueError, match="ROCm"):
        solve(torch.rand(3, 3), reg=0.1, n_iter=5)


@pytest.mark.parametrize(("N", "M"), [(3, 5), (4, 128)], ids=["two-sweep", "fused"])
def test_batch_above_grid_limit(N, M, device):
    """70,000 problems: the launches that put the batch on a grid dimension
    (prepare, the fused step and its merge, the column sweep) run in slices."""
    B = 70_000
    cost = torch.rand(B, N, M, generator=torch.Generator().manual_seed(22))
    a = workloads.uniform_marginal(B, N)
    b = workloads.uniform_marginal(B, M)
    r32 = sk.log_sinkhorn_plan(cost, eps=0.1, n_iter=8, a=a, b=b)
    r64 = sk.log_sinkhorn_plan(cost, eps=0.1, n_iter=8, a=a, b=b, dtype=torch.float64)
    plan = torch.ops.transport.log_sinkhorn(cost.to(device), 0.1, 8, a.to(device), b.to(device))
    sk_parity.check(f"B={B} {(N, M)}", {"plan": plan}, {"plan": r32[0]}, {"plan": r64[0]})
