"""The fused preparation pass of the gfx950 Sinkhorn (mask, validation,
largest finite cost, all-+inf rows / columns) against what the reference
computes with separate torch passes (transport/matrix/_validate.py:19-156,
_schedule.py:68-69, _log_sinkhorn.py:36-46).

* A mask fused in the kernels gives the bits of the op run on the cost the
  reference's ``masked_fill(~mask, inf)`` materialises: the log kernel of a
  masked pair is -inf either way, so the two runs are identical.
* NaN / -inf in the cost (also under a masked pair: the reference validates
  before fusing) and negative marginals raise the reference's exceptions.
* The schedule built from the device maximum equals the one the reference
  builds from the cost (negative costs, +inf, masked maxima, nothing finite).
* The C entry points report the flags and the maximum bit-exactly.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

import torchmatch_amd  # noqa: F401
from torchmatch_amd import _native
import workloads
from torchmatch_amd.transport.matrix import Backend, solve
from torchmatch_amd.transport.matrix._schedule import build_eps_schedule
from torchmatch_amd.transport.matrix._sinkhorn import _device_solve, log_sinkhorn_plan

pytestmark = pytest.mark.gpu

INF = float("inf")


def _masked_problem(B, N, M, seed, drop=0.2):
    g = torch.Generator().manual_seed(seed)
    cost = workloads.sinkhorn_points(B, N, M, 8, seed=seed)
    mask = torch.rand(B, N, M, generator=g) > drop
    mask[:, 1, :] = False                 # a fully masked row
    mask[:, :, 2] = False                 # and column
    a = workloads.uniform_marginal(B, N)
    b = workloads.uniform_marginal(B, M)
    return cost, mask, a, b


@pytest.mark.parametrize(("B", "N", "M"), [
    (2, 50, 60),      # float4 pass
    (2, 33, 37),      # scalar pass (M % 4 != 0)
    (1, 48, 4100),    # long rows
    (3, 300, 200),
])
def test_mask_fused_matches_materialised(B, N, M, device):
    cost, mask, a, b = _masked_problem(B, N, M, seed=N + M)
    cd, md, ad, bd = (t.to(device) for t in (cost, mask, a, b))
    fused = torch.ops.transport.log_sinkhorn(cd, 0.1, 40, ad, bd, md)
    materialised = torch.ops.transport.log_sinkhorn(cd.masked_fill(~md, INF), 0.1, 40, ad, bd)
    print(f"mask fused {(B, N, M)} equal {torch.equal(fused, materialised)}", flush=True)
    assert torch.equal(fused, materialised)
    assert torch.isneginf(fused[:, 1, :]).all() and torch.isneginf(fused[:, :, 2]).all()
    ub = torch.ops.transport.unbalanced_sinkhorn(cd, 0.1, 30, 0.5, ad, bd, md)
    ub_ref = torch.ops.transport.unbalanced_sinkhorn(cd.masked_fill(~md, INF), 0.1, 30, 0.5,
                                                     ad, bd)
    assert torch.equal(ub, ub_ref)


def test_broadcast_mask_and_scaling(device):
    cost, mask, a, b = _masked_problem(3, 40, 44, seed=3)
    per_pair = mask[0].to(device)
    cd, ad, bd = cost.to(device), a.to(device), b.to(device)
    got = torch.ops.transport.log_sinkhorn(cd, 0.05, 60, ad, bd, per_pair, 0.6)
    want = torch.ops.transport.log_sinkhorn(cd.masked_fill(~per_pair, INF), 0.05, 60, ad, bd,
                                            None, 0.6)
    assert torch.equal(got, want)
    via_solve = solve(cd, reg=0.05, n_iter=60, a=ad, b=bd, mask=per_pair, scaling=0.6)
    assert torch.equal(via_solve, want)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_nan_and_neg_inf_raise(dtype, device):
    cost = torch.rand(2, 30, 40, dtype=dtype, device=device)
    a = torch.full((2, 30), 1 / 30, dtype=dtype, device=device)
    b = torch.full((2, 40), 1 / 40, dtype=dtype, device=device)
    bad = cost.clone()
    bad[1, 17, 33] = float("nan")
    with pytest.raises(RuntimeError, match="cost contains NaN"):
        torch.ops.transport.log_sinkhorn(bad, 0.1, 5, a, b)
    with pytest.raises(RuntimeError, match="cost contains NaN"):
        solve(bad, reg=0.1, n_iter=5, backend=Backend.UNBALANCED_SINKHORN)
    # validated before the mask is fused: a masked NaN still raises
    mask = torch.ones_like(bad, dtype=torch.bool)
    mask[1, 17, 33] = False
    with pytest.raises(RuntimeError, match="cost contains NaN"):
        torch.ops.transport.log_sinkhorn(bad, 0.1, 5, a, b, mask)
    bad = cost.clone()
    bad[0, 0, 39] = -INF
    with pytest.raises(RuntimeError, match="cost contains -inf"):
        torch.ops.transport.sinkhorn_divergence(bad, 0.1, 5, a, b)
    bad[0, 3, 3] = float("nan")
    with pytest.raises(RuntimeError, match="cost contains NaN"):
        torch.ops.transport.unbalanced_sinkhorn(bad, 0.1, 5, 1.0, a, b)
    # +inf is a forbidden pair, not an error
    ok = cost.clone()
    ok[0, 5, :] = INF
    plan = torch.ops.transport.log_sinkhorn(ok, 0.1, 5, a, b)
    assert torch.isneginf(plan[0, 5]).all()


def test_error_order_matches_reference(device):
    cost = torch.rand(2, 6, 5, device=device)
    a = torch.full((2, 6), 1 / 6, device=device)
    b = torch.full((2, 5), 1 / 5, device=device)
    neg_a = a.clone()
    neg_a[1, 2] = -0.01
    neg_b = b.clone()
    neg_b[0, 0] = -0.5
    with pytest.raises(ValueError, match="a must be non-negative"):
        solve(cost, a=neg_a, b=neg_b, reg=0.1, n_iter=5)
    with pytest.raises(ValueError, match="b must be non-negative"):
        solve(cost, a=a, b=neg_b, reg=0.1, n_iter=5, backend="sinkhorn_divergence")
    nan_cost = cost.clone()
    nan_cost[0, 0, 0] = float("nan")
    with pytest.raises(RuntimeError, match="cost contains NaN"):
        solve(nan_cost, a=neg_a, reg=0.1, n_iter=5)
    # cost checks come before the schedule's own argument checks
    with pytest.raises(RuntimeError, match="cost contains NaN"):
        torch.ops.transport.log_sinkhorn(nan_cost, -1.0, 5, a, b)
    with pytest.raises(ValueError, match="reg must be positive"):
        torch.ops.transport.log_sinkhorn(cost, -1.0, 5, a, b)
    with pytest.raises(ValueError, match="rho must be positive"):
        torch.ops.transport.unbalanced_sinkhorn(cost, 0.1, 5, 0.0, a, b)
    with pytest.raises(RuntimeError, match="cost contains NaN"):
        torch.ops.transport.unbalanced_sinkhorn(nan_cost, 0.1, 5, 0.0, a, b)
    with pytest.raises(ValueError, match="rho must be positive for UNBALANCED_SINKHORN"):
        solve(cost, backend="unbalanced_sinkhorn", reg=0.1, n_iter=5, rho=-1.0)


@pytest.mark.parametrize("case", ["plain", "negative", "inf", "masked_max", "all_inf"])
def test_schedule_from_device_max(case, device):
    g = torch.Generator().manual_seed(9)
    cost = torch.rand(3, 70, 90, generator=g) * 4.0
    mask = None
    if case == "negative":
        cost = cost - 10.0
    elif case == "inf":
        cost[cost > 3.5] = INF
    elif case == "masked_max":
        cost[2, 5, 7] = 100.0
        mask = torch.ones(3, 70, 90, dtype=torch.bool)
        mask[2, 5, 7] = False
    elif case == "all_inf":
        cost = torch.full((3, 70, 90), INF)
    a = torch.full((3, 70), 1 / 70)
    b = torch.full((3, 90), 1 / 90)
    fused = cost if mask is None else cost.masked_fill(~mask, INF)
    want = build_eps_schedule(cost=fused, reg=0.01, n_iter=30, scaling=0.8)
    got, *_ = _device_solve(
        cost.to(device), a.to(device), b.to(device), eps=0.01, n_iter=30, scaling=0.8,
        rho=0.0, who="test", mask=None if mask is None else mask.to(device), check_cost=True,
    )
    assert got == want


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


@pytest.mark.parametrize("vec", [True, False])
def test_c_abi_prepare_reports_flags_and_max(vec, device):
    lib = _native.lib()
    B, N, M = 2, 67, (64 if vec else 61)
    g = torch.Generator().manual_seed(4)
    cost = torch.randn(B, N, M, generator=g)
    cost[1, 66, M - 1] = 7.25          # largest finite, at the last row / column
    cost[0, 3, 5] = INF
    a = torch.rand(B, N, generator=g)
    b = torch.rand(B, M, generator=g)
    ws = torch.empty(lib.tm_sinkhorn_workspace_bytes(B, N, M), dtype=torch.uint8, device=device)
    stream = ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)

    def stats(c, keep=None, a_=a, b_=b):
        cd, ad, bd = c.to(device), a_.to(device), b_.to(device)
        kd = None if keep is None else keep.to(device)
        rc = lib.tm_sinkhorn_prepare_f32(_ptr(cd), None if kd is None else _ptr(kd), _ptr(ad),
                                         _ptr(bd), B, N, M, 0.0, _ptr(ws), ws.numel(), stream)
        assert rc == _native.TM_OK
        flags, mx = ctypes.c_uint32(0), ctypes.c_float(0.0)
        rc = lib.tm_sinkhorn_read_stats(_ptr(ws), B, N, M, ctypes.byref(flags),
                                        ctypes.byref(mx), stream)
        assert rc == _native.TM_OK
        return flags.value, mx.value

    assert stats(cost) == (16, 7.25)
    keep = torch.ones(B, N, M, dtype=torch.bool)
    keep[1, 66, M - 1] = False
    fin = cost.masked_fill(~keep, INF)
    assert stats(cost, keep) == (16, fin[torch.isfinite(fin)].max().item())
    bad = cost.clone()
    bad[0, 10, 1] = float("nan")
    bad[1, 0, 0] = -INF
    neg_a, neg_b = a.clone(), b.clone()
    neg_a[1, 5] = -1e-30
    neg_b[0, M - 1] = -2.0
    flags, _ = stats(bad, None, neg_a, neg_b)
    assert flags == 1 | 2 | 4 | 8 | 16
    assert stats(torch.full((B, N, M), INF)) == (0, -INF)


def test_zero_size_potentials(device):
    cost = torch.empty(2, 0, 5, device=device)
    plan, f, g = log_sinkhorn_plan(cost, eps=0.1, n_iter=3, a=torch.empty(2, 0, device=device),
                                   b=torch.full((2, 5), 0.2, device=device),
                                   return_potentials=True)
    assert plan.shape == (2, 0, 5) and f.shape == (2, 0)
    assert torch.equal(g, torch.zeros(2, 5, device=device))


_GUARD_SCRIPT = """
import sys
sys.path.insert(0, {root!r})
import torch
import torchmatch_amd  # noqa: F401
cost = torch.rand(2, 16, 16, device="cuda")
a = torch.full((2, 16), 1 / 16, device="cuda")
graph = torch.cuda.CUDAGraph()
try:
    with torch.cuda.graph(graph):
        torch.ops.transport.log_sinkhorn(cost, 0.1, 5, a, a)
except RuntimeError as exc:
    message = str(exc)
    print("GUARD_RAISED_OK" if "CUDA graph capture" in message else "WRONG: " + message)
    sys.exit(0)
print("GUARD_DID_NOT_RAISE")
sys.exit(1)
"""


def test_graph_capture_guard(device):
    """The validation readback cannot run under stream capture: the op says
    so (as the JV op does, assignment/cuda/dispatch.cu:97-106) instead of
    failing inside the capture."""
    import subprocess
    import sys
    from pathlib import Path

    root = str(Path(__file__).resolve().parents[1])
    res = subprocess.run([sys.executable, "-c", _GUARD_SCRIPT.format(root=root)],
                         capture_output=True, text=True, timeout=120)
    assert "GUARD_RAISED_OK" in res.stdout, f"{res.stdout!r} {res.stderr[-2000:]!r}"
