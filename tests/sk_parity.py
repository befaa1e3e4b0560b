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

Every quantity is held to the north star's 1e-5 (``ELEM_BOUND``).  The
figures printed beside it say how far float32 itself moves the quantity: the
reference's own float32 result differs from the same recurrence in float64 by
``drift`` (the oracle run at both precisions), and the kernel's distance from
float64 is printed too.  The full-size tests additionally require the
kernel's potentials to be no further from float64 than the reference's are
(``check_vs_f64``).
"""

from __future__ import annotations

import torch

ELEM_BOUND = 1e-5   # north star: 1e-5 relative per plan entry and per potential


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


def check(label: str, got: dict, ref32: dict, ref64: dict) -> dict:
    """Compare each named quantity (``plan`` = log plan, or a potential) of the
    kernels with the float32 oracle: max-abs within ELEM_BOUND.  Prints the
    error, the kernel's distance from the float64 oracle and the float32
    oracle's own drift from float64; returns (err, err64, drift) per name."""
    out = {}
    for name, x in got.items():
        err = logp_err(x, ref32[name])
        drift = logp_err(ref32[name], ref64[name])
        err64 = logp_err(x, ref64[name])
        out[name] = (err, err64, drift)
        print(f"  {label} {name}: max-abs vs oracle f32 {err:.3e}, vs f64 {err64:.3e}, "
              f"oracle f32 drift {drift:.3e}, bound {ELEM_BOUND:.0e}", flush=True)
    for name, (err, _, _) in out.items():
        assert err <= ELEM_BOUND, f"{label} {name}: {err:.3e} > {ELEM_BOUND:.0e}"
    return out


def check_vs_f64(label: str, err64: float, drift: float) -> None:
    """The kernel's potential is no further from the float64 recurrence than
    the reference's own float32 result is."""
    assert err64 <= drift, (f"{label}: {err64:.3e} from float64, further than the "
                            f"reference's float32 drift {drift:.3e}")
