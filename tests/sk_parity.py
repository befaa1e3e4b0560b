"""Element-wise parity measures shared by the Sinkhorn GPU tests.

North star: plans and potentials within 1e-5 relative of the reference, the
max-abs error reported.  The relative error of a plan entry P = exp(log P)
is |exp(d) - 1| ~ |d| with d = log P - log P_ref, so the plan measure is
element-wise on the log plan:

* ``logp_err``: max |log P - log P_ref| over the entries that are finite in
  the reference, after checking that the -inf pattern (forbidden cells, empty
  rows / columns) is identical and that nothing is NaN;
* ``pot_err``: max-abs error of a potential (f, g, log_u or log_v) over its
  finite entries, same pattern check.

float32 itself moves these quantities: the reference's own float32 result
differs from the same recurrence in float64 by ``drift`` (measured per case
by running the oracle at both precisions).  A second float32 computation with
another summation order (the kernels) can differ from the reference by up to
about twice that, so the bound is ``max(ELEM_FLOOR, ELEM_K * drift)``.
"""

from __future__ import annotations

import torch

ELEM_FLOOR = 1e-5   # north star: 1e-5 relative per plan entry
ELEM_K = 2.5        # kernel vs reference: two independent float32 roundings of one recurrence


def _check_pattern(x: torch.Tensor, ref: torch.Tensor) -> torch.Tensor:
    assert not torch.isnan(x).any(), "NaN in the result"
    assert torch.equal(torch.isneginf(x), torch.isneginf(ref)), "-inf pattern differs"
    fin = torch.isfinite(ref)
    assert torch.equal(fin, torch.isfinite(x)), "finite pattern differs"
    return fin


def logp_err(log_plan: torch.Tensor, ref: torch.Tensor) -> float:
    """max |log P - log P_ref| over finite reference entries (CPU, float64)."""
    x, r = log_plan.detach().cpu().double(), ref.detach().cpu().double()
    fin = _check_pattern(x, r)
    if not fin.any():
        return 0.0
    return (x[fin] - r[fin]).abs().max().item()


def pot_err(x: torch.Tensor, ref: torch.Tensor) -> float:
    """max-abs error of a potential over its finite reference entries."""
    return logp_err(x, ref)


def bound(drift: float) -> float:
    return max(ELEM_FLOOR, ELEM_K * drift)


def check(label: str, got: dict, ref32: dict, ref64: dict) -> dict:
    """Compare each named quantity (``plan`` = log plan, or a potential) of the
    kernels with the float32 oracle, bounded by the oracle's own float32 vs
    float64 drift on the same input.  Prints every figure; returns them."""
    out = {}
    for name, x in got.items():
        err = logp_err(x, ref32[name])
        drift = logp_err(ref32[name], ref64[name])
        err64 = logp_err(x, ref64[name])
        out[name] = (err, drift)
        print(f"  {label} {name}: max-abs vs oracle f32 {err:.3e}, vs f64 {err64:.3e}, "
              f"oracle f32 drift {drift:.3e}, bound {bound(drift):.3e}", flush=True)
    for name, (err, drift) in out.items():
        assert err <= bound(drift), f"{label} {name}: {err:.3e} > {bound(drift):.3e}"
    return out
