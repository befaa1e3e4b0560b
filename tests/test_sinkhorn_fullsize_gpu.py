"""Full-size Sinkhorn parity: C4 (log_sinkhorn) and C5 (unbalanced_sinkhorn).

The fixtures come from ``tests/golden/make_sinkhorn_golden.py``, which ran
the CPU oracle (the reference's torch calls in their order,
``_log_sinkhorn.py:136-221`` / ``_unbalanced_sinkhorn.py:30-103``) on the
exact configurations of BASELINE.json:

* C4: (16, 2048, 2048) squared distances of seeded N(0, I_8) clouds over
  their global max, uniform marginals, reg 0.05, 200 iterations;
* C5: (1, 16384, 16384) built the same way, Dirichlet(1) marginals of total
  mass 1.0 and 1.3, reg 0.02, rho 1.0, 500 iterations.

Each test regenerates the input on the CPU (sha256 checked against the
fixture), runs the kernels, and compares

* the potentials log_u, log_v with the oracle's float32 ones (max-abs);
* every entry of the log plan with the oracle's plan, rebuilt bit for bit
  from the stored potentials and the cost, (log_u + (-C / eps)) + log_v, the
  reference's float32 expression: max |log P - log P_ref| over finite entries.

Both are held to the north star's 1e-5.  The potentials must also be no
further from the float64 recurrence (the fixture's log_u64 / log_v64) than
the reference's own float32 result is: the fixture records that drift for the
same input.  C4 also re-runs the oracle here, on this machine's torch, and
holds the kernels to that run as well.
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch

import sk_parity
import torchmatch_amd  # noqa: F401
from oracle import sinkhorn as sk
import workloads
from torchmatch_amd.transport.matrix import _sinkhorn

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
INDEX = json.loads((GOLDEN / "sk_golden.json").read_text())


def _marginal(spec: dict, B: int, n: int) -> torch.Tensor:
    if spec["kind"] == "uniform":
        return workloads.uniform_marginal(B, n)
    return workloads.dirichlet(B, n, spec["total"], seed=spec["seed"])


def _inputs(case: dict):
    B, N, M = case["B"], case["N"], case["M"]
    cost = workloads.sinkhorn_points(B, N, M, case["D"], seed=case["cost_seed"])
    a, b = _marginal(case["a"], B, N), _marginal(case["b"], B, M)
    for name, t in (("cost", cost), ("a", a), ("b", b)):
        assert workloads.sha256(t) == case["sha256"][name], f"{name} bytes differ from fixture"
    return cost, a, b


def _fixture(case: dict) -> dict:
    with np.load(GOLDEN / case["file"]) as z:
        return {k: torch.from_numpy(z[k]) for k in z.files}


def _plan_err(plan_dev: torch.Tensor, cost: torch.Tensor, log_u: torch.Tensor,
              log_v: torch.Tensor, eps: float, chunk: int = 1024) -> float:
    """max |log P - log P_ref| over the reference's finite entries, the
    reference plan rebuilt by row chunks from its float32 potentials."""
    worst = 0.0
    n = cost.shape[1]
    for i0 in range(0, n, chunk):
        rows = slice(i0, min(n, i0 + chunk))
        ref = (log_u[:, rows, None] + (-cost[:, rows] / eps)) + log_v[:, None, :]
        got = plan_dev[:, rows].cpu()
        worst = max(worst, sk_parity.logp_err(got, ref))
    return worst


def _run_device(case: dict, cost, a, b, device):
    """The kernels' plan through the public op, and the potentials of the
    same solve through the internal entry the op wraps (bit-identical plan)."""
    cd, ad, bd = cost.to(device), a.to(device), b.to(device)
    eps, n_iter = case["reg"], case["n_iter"]
    if case["rho"] is None:
        plan = torch.ops.transport.log_sinkhorn(cd, eps, n_iter, ad, bd)
        rho = 0.0
    else:
        plan = torch.ops.transport.unbalanced_sinkhorn(cd, eps, n_iter, case["rho"], ad, bd)
        rho = float(case["rho"])
    _, plan2, log_u, log_v = _sinkhorn._device_solve(
        cd, ad, bd, eps=eps, n_iter=n_iter, scaling=None, rho=rho, who="fullsize")
    torch.cuda.synchronize()
    assert torch.equal(plan, plan2), "op and internal solve disagree"
    del plan2, cd
    return plan, log_u.cpu(), log_v.cpu()


def _check(name: str, case: dict, plan, log_u, log_v, cost, fx: dict) -> None:
    drift = case["drift_f32_vs_f64"]
    eps = case["reg"]
    eu = sk_parity.pot_err(log_u, fx["log_u"])
    ev = sk_parity.pot_err(log_v, fx["log_v"])
    eu64 = sk_parity.pot_err(log_u, fx["log_u64"])
    ev64 = sk_parity.pot_err(log_v, fx["log_v64"])
    ep = _plan_err(plan, cost, fx["log_u"], fx["log_v"], eps)
    print(f"{name}: log_u max-abs {eu:.3e} (vs f64 {eu64:.3e}, oracle drift {drift['log_u']:.3e})"
          f"; log_v {ev:.3e} (vs f64 {ev64:.3e}, drift {drift['log_v']:.3e})"
          f"; log plan element-wise {ep:.3e} (drift {drift['log_plan_elementwise']:.3e})",
          flush=True)
    for label, err in (("log_u", eu), ("log_v", ev), ("log plan element-wise", ep)):
        assert err <= sk_parity.ELEM_BOUND, f"{name} {label}: {err:.3e} > 1e-5"
    sk_parity.check_vs_f64(f"{name} log_u", eu64, drift["log_u"])
    sk_parity.check_vs_f64(f"{name} log_v", ev64, drift["log_v"])


def test_c4_full_size_matches_oracle(device):
    case = INDEX["c4"]
    print("C4 full size: building input", flush=True)
    cost, a, b = _inputs(case)
    fx = _fixture(case)
    plan, log_u, log_v = _run_device(case, cost, a, b, device)
    _check("C4 vs fixture", case, plan, log_u, log_v, cost, fx)
    # the oracle again, on this machine's torch build
    print("C4 full size: CPU oracle (200 iterations)", flush=True)
    _, _, _, ou, ov = sk.log_sinkhorn_plan(cost, eps=case["reg"], n_iter=case["n_iter"],
                                           a=a, b=b)
    here = {"log_u": ou, "log_v": ov, "log_u64": fx["log_u64"], "log_v64": fx["log_v64"]}
    print(f"  oracle here vs fixture: log_u {sk_parity.pot_err(ou, fx['log_u']):.3e}, "
          f"log_v {sk_parity.pot_err(ov, fx['log_v']):.3e}", flush=True)
    _check("C4 vs oracle here", case, plan, log_u, log_v, cost, here)


def test_c5_full_size_matches_oracle(device):
    case = INDEX["c5"]
    print("C5 full size: building input", flush=True)
    cost, a, b = _inputs(case)
    fx = _fixture(case)
    plan, log_u, log_v = _run_device(case, cost, a, b, device)
    _check("C5 vs fixture", case, plan, log_u, log_v, cost, fx)
