"""Write the full-size Sinkhorn parity fixtures (C4 and C5) from the CPU oracle.

Runs in the build container (about 30 GiB of RAM at C5, float64 included):

    python tests/golden/make_sinkhorn_golden.py [c4] [c5]

``oracle/sinkhorn.py`` restates the reference's torch calls in their order
(``transport/matrix/_log_sinkhorn.py:136-221`` for C4,
``_unbalanced_sinkhorn.py:30-103`` for C5).  For each configuration the
fixture holds:

* the input recipe (generator, shape, seeds) and the sha256 of the float32
  cost and marginal bytes, so a test regenerates the exact input;
* the oracle's final potentials ``log_u`` / ``log_v`` in float32 (the
  reference's arithmetic) and in float64 (the same recurrence at double
  precision, the yardstick for how far float32 itself drifts).

The oracle's log plan is ``(log_u[:, :, None] + (-cost / eps)) + log_v[:, None, :]``
in float32 (``_log_sinkhorn.py:217``, ``_unbalanced_sinkhorn.py:101-103``), so
any plan entry is rebuilt bit-for-bit from the stored potentials and the
regenerated cost; this script checks that rebuild against the plan the oracle
returned.  ``sk_golden.json`` records, per configuration, the element-wise
drift of the float32 oracle from the float64 one: max |log P32 - log P64|
over finite entries (the relative error of each plan entry) and max-abs of
the potentials.  The GPU tests bound their own error by that drift.
"""

from __future__ import annotations

import json
import sys
import time
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import sinkhorn as sk  # noqa: E402
import workloads  # noqa: E402

OUT = Path(__file__).resolve().parent
INDEX = OUT / "sk_golden.json"

CASES: dict[str, dict] = {
    "c4": {
        "op": "log_sinkhorn",
        "B": 16, "N": 2048, "M": 2048, "D": 8, "cost_seed": 0,
        "a": {"kind": "uniform"}, "b": {"kind": "uniform"},
        "reg": 0.05, "n_iter": 200, "rho": None,
        "file": "sk_c4_16x2048x2048.npz",
    },
    "c5": {
        "op": "unbalanced_sinkhorn",
        "B": 1, "N": 16384, "M": 16384, "D": 8, "cost_seed": 0,
        "a": {"kind": "dirichlet", "total": 1.0, "seed": 1},
        "b": {"kind": "dirichlet", "total": 1.3, "seed": 2},
        "reg": 0.02, "n_iter": 500, "rho": 1.0,
        "file": "sk_c5_1x16384x16384.npz",
    },
}


def marginal(spec: dict, B: int, n: int) -> torch.Tensor:
    if spec["kind"] == "uniform":
        return workloads.uniform_marginal(B, n)
    return workloads.dirichlet(B, n, spec["total"], seed=spec["seed"])


def make_inputs(case: dict) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    B, N, M = case["B"], case["N"], case["M"]
    cost = workloads.sinkhorn_points(B, N, M, case["D"], seed=case["cost_seed"])
    return cost, marginal(case["a"], B, N), marginal(case["b"], B, M)


def plan_rows(cost, log_u, log_v, eps, rows):
    """Rows ``rows`` of the oracle's log plan, the same float ops in the same
    order as the oracle (and the reference)."""
    c = cost[:, rows].to(log_u.dtype)
    return (log_u[:, rows, None] + (-c / eps)) + log_v[:, None, :]


def run(case: dict, dtype: torch.dtype, cost, a, b):
    kw = dict(eps=case["reg"], n_iter=case["n_iter"], a=a, b=b, dtype=dtype)
    if case["rho"] is None:
        plan, _, _, log_u, log_v = sk.log_sinkhorn_plan(cost, **kw)
    else:
        plan, log_u, log_v = sk.unbalanced_sinkhorn_plan(cost, rho=case["rho"], **kw)
    return plan, log_u, log_v


def drift(cost, eps, pot32, pot64, chunk: int = 512) -> float:
    """max |log P32 - log P64| over entries finite in both, by row chunks."""
    worst = 0.0
    n = cost.shape[1]
    for i0 in range(0, n, chunk):
        rows = slice(i0, min(n, i0 + chunk))
        p32 = plan_rows(cost, *pot32, eps, rows).double()
        p64 = plan_rows(cost, *pot64, eps, rows)
        fin = torch.isfinite(p32) & torch.isfinite(p64)
        if fin.any():
            worst = max(worst, (p32[fin] - p64[fin]).abs().max().item())
    return worst


def make(name: str) -> dict:
    case = CASES[name]
    cost, a, b = make_inputs(case)
    eps = case["reg"]
    print(f"{name}: cost {tuple(cost.shape)} sha256 {workloads.sha256(cost)[:16]}", flush=True)
    t0 = time.perf_counter()
    plan32, lu32, lv32 = run(case, torch.float32, cost, a, b)
    t32 = time.perf_counter() - t0
    # the stored potentials rebuild the oracle's plan bit for bit
    n = cost.shape[1]
    for rows in (slice(0, 64), slice(n - 64, n)):
        assert torch.equal(plan_rows(cost, lu32, lv32, eps, rows), plan32[:, rows]), \
            "plan rebuild from potentials is not bit-identical"
    del plan32
    print(f"  float32 oracle {t32:.1f} s", flush=True)
    t0 = time.perf_counter()
    plan64, lu64, lv64 = run(case, torch.float64, cost, a, b)
    t64 = time.perf_counter() - t0
    del plan64
    print(f"  float64 oracle {t64:.1f} s", flush=True)
    d_plan = drift(cost, eps, (lu32, lv32), (lu64, lv64))

    def pot_drift(x32, x64):
        fin = torch.isfinite(x64)
        return (x32.double()[fin] - x64[fin]).abs().max().item() if fin.any() else 0.0

    np.savez_compressed(
        OUT / case["file"],
        log_u=lu32.numpy(), log_v=lv32.numpy(),
        log_u64=lu64.numpy(), log_v64=lv64.numpy(),
    )
    entry = {
        **case,
        "sha256": {"cost": workloads.sha256(cost), "a": workloads.sha256(a),
                   "b": workloads.sha256(b)},
        "drift_f32_vs_f64": {
            "log_plan_elementwise": d_plan,
            "log_u": pot_drift(lu32, lu64),
            "log_v": pot_drift(lv32, lv64),
            "max_abs_log_plan": max(
                plan_rows(cost, lu64, lv64, eps, slice(0, 64)).abs()
                .nan_to_num(posinf=0, neginf=0).max().item(), 0.0),
        },
        "oracle_seconds": {"float32": round(t32, 1), "float64": round(t64, 1),
                           "threads": torch.get_num_threads()},
        "torch": torch.__version__,
    }
    print(f"  drift: {entry['drift_f32_vs_f64']}", flush=True)
    return entry


def main() -> None:
    names = [a for a in sys.argv[1:] if a in CASES] or list(CASES)
    index = json.loads(INDEX.read_text()) if INDEX.exists() else {}
    for name in names:
        index[name] = make(name)
        INDEX.write_text(json.dumps(index, indent=2) + "\n")


if __name__ == "__main__":
    main()
