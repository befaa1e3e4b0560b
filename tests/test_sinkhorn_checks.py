"""Host side of the fused Sinkhorn checks -- no GPU needed.

The device preparation pass reports NaN / -inf in the cost, negative
marginals and the largest finite cost as flags; these tests pin the host
logic around it against the reference's rules
(transport/matrix/_validate.py:19-156, _schedule.py:21-76):

* the flags raise the reference's exceptions and messages in its order;
* the schedule built from a measured maximum equals the one built from the
  cost (and the oracle's);
* the mask operand is the broadcast ``masked_fill`` applies, or None;
* solve() keeps the reference's error order when the marginal shapes are
  wrong as well (the torch path re-checks in order);
* the C entry points reject bad arguments before any GPU work.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

import torchmatch_amd  # noqa: F401
from oracle import sinkhorn as sk
from torchmatch_amd import _native
from torchmatch_amd.transport.matrix import solve
from torchmatch_amd.transport.matrix._schedule import build_eps_schedule, schedule_from_max
from torchmatch_amd.transport.matrix._validate import (
    FLAG_A_NEG,
    FLAG_B_NEG,
    FLAG_NAN,
    FLAG_NEG_INF,
    kernel_keep_mask,
    raise_for_flags,
)


@pytest.mark.parametrize(("flags", "exc", "msg"), [
    (FLAG_NAN | FLAG_NEG_INF | FLAG_A_NEG, RuntimeError, "cost contains NaN"),
    (FLAG_NEG_INF | FLAG_B_NEG, RuntimeError, "cost contains -inf"),
    (FLAG_A_NEG | FLAG_B_NEG, ValueError, "a must be non-negative"),
    (FLAG_B_NEG, ValueError, "b must be non-negative"),
])
def test_flags_raise_in_reference_order(flags, exc, msg):
    with pytest.raises(exc, match=msg):
        raise_for_flags(flags, cost=True, marginals=True)


def test_flags_only_checked_when_asked():
    raise_for_flags(FLAG_NAN | FLAG_NEG_INF, cost=False, marginals=True)
    raise_for_flags(FLAG_A_NEG | FLAG_B_NEG, cost=True, marginals=False)
    with pytest.raises(ValueError, match="a must be"):
        raise_for_flags(FLAG_NAN | FLAG_A_NEG, cost=False, marginals=True)


@pytest.mark.parametrize("cost", [
    torch.tensor([[0.0, 4.0], [1.0, float("inf")]]),
    torch.tensor([[-3.0, -0.5], [-7.0, float("inf")]]),   # negative largest value
    torch.full((2, 3), float("inf")),                      # nothing finite
    torch.tensor([[0.25]]),                                # below reg after halving
])
@pytest.mark.parametrize("scaling", [None, 0.5, 0.9])
def test_schedule_from_max_matches_cost_schedule(cost, scaling):
    fin = cost[torch.isfinite(cost)]
    max_finite = fin.max().item() if fin.numel() else None
    got = schedule_from_max(reg=0.1, n_iter=40, scaling=scaling, max_finite=max_finite)
    assert got == build_eps_schedule(cost=cost, reg=0.1, n_iter=40, scaling=scaling)
    assert got == sk.eps_schedule(cost, 0.1, 40, scaling)


@pytest.mark.parametrize(("kw", "msg"), [
    ({"reg": -1.0, "n_iter": 3, "scaling": None}, "reg must be positive"),
    ({"reg": 0.1, "n_iter": 0, "scaling": 0.5}, "n_iter must be >= 1"),
    ({"reg": 0.1, "n_iter": 3, "scaling": 0.0}, "scaling must be in"),
])
def test_schedule_from_max_errors(kw, msg):
    with pytest.raises(ValueError, match=msg):
        schedule_from_max(max_finite=1.0, **kw)


def test_keep_mask_operand():
    cost = torch.rand(3, 4, 5)
    same = torch.rand(3, 4, 5) > 0.5
    assert kernel_keep_mask(cost, same).data_ptr() == same.data_ptr()
    per_pair = torch.rand(4, 5) > 0.5
    keep = kernel_keep_mask(cost, per_pair)
    assert keep.shape == cost.shape and keep.is_contiguous()
    assert torch.equal(keep, per_pair.expand(3, 4, 5))
    assert kernel_keep_mask(cost, per_pair.float()) is None        # not bool
    assert kernel_keep_mask(cost, torch.ones(2, 4, 5, dtype=torch.bool)) is None
    # the fallback raises what torch's masked_fill raises for such masks
    with pytest.raises((RuntimeError, TypeError)):
        cost.masked_fill(~per_pair.float(), float("inf"))


def test_solve_error_order_with_bad_shapes():
    """validate_cost before coerce_marginals, a before b (_solve.py:98-140)."""
    cost = torch.rand(3, 4)
    cost[1, 2] = float("nan")
    with pytest.raises(RuntimeError, match="cost contains NaN"):
        solve(cost, a=torch.ones(7), reg=0.1, n_iter=3)
    cost = torch.rand(3, 4)
    a = torch.tensor([0.5, -0.1, 0.6])
    with pytest.raises(ValueError, match="a must be non-negative"):
        solve(cost, a=a, b=torch.ones(9), reg=0.1, n_iter=3)
    with pytest.raises(ValueError, match=r"b must have shape"):
        solve(cost, a=a.abs(), b=torch.ones(9), reg=0.1, n_iter=3)


def test_c_entry_points_reject_bad_arguments():
    lib = _native.lib()
    bad, ok = _native.TM_ERR_INVALID_ARGUMENT, _native.TM_OK
    assert lib.tm_sinkhorn_prepare_f32(None, None, None, None, -1, 4, 4, 0.1, None, 0,
                                       None) == bad
    assert lib.tm_sinkhorn_prepare_f32(None, None, None, None, 1, 4, 4, -0.5, None, 0,
                                       None) == bad
    assert lib.tm_sinkhorn_prepare_f32(None, None, None, None, 0, 4, 4, 0.1, None, 0,
                                       None) == ok   # empty: nothing launched
    flags, mx = ctypes.c_uint32(7), ctypes.c_float(3.0)
    assert lib.tm_sinkhorn_read_stats(None, 2, 0, 4, ctypes.byref(flags), ctypes.byref(mx),
                                      None) == ok
    assert flags.value == 0 and mx.value == float("-inf")
    sched = (ctypes.c_double * 2)(0.1, 0.1)
    assert lib.tm_sinkhorn_iterate_f32(None, None, 1, 4, 4, sched, 0, 0.0, 0.0, None, None,
                                       None, None, 0, None) == bad
    sched[1] = 0.0
    assert lib.tm_sinkhorn_iterate_f32(None, None, 1, 4, 4, sched, 2, 0.0, 0.0, None, None,
                                       None, None, 0, None) == bad
    assert lib.tm_sinkhorn_iterate_f32(None, None, 0, 4, 4, sched, 1, 0.0, 0.0, None, None,
                                       None, None, 0, None) == ok


def test_private_op_schemas():
    assert str(torch.ops.torchmatch_amd.sinkhorn_prepare.default._schema) == (
        "torchmatch_amd::sinkhorn_prepare(Tensor cost, Tensor? keep, Tensor a, Tensor b, "
        "float k_eps, bool read_stats) -> (Tensor, Tensor)"
    )
    assert str(torch.ops.torchmatch_amd.sinkhorn_iterate.default._schema) == (
        "torchmatch_amd::sinkhorn_iterate(Tensor cost, Tensor? keep, Tensor ws, "
        "float[] eps_sched, float rho, float k_eps, bool write_plan) -> "
        "(Tensor, Tensor, Tensor)"
    )
