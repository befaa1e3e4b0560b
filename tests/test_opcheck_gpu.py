"""``torch.library.opcheck`` on the device registrations of every public op.

The reference runs opcheck with ``test_schema`` + ``test_faketensor`` on its
CUDA JV op and on the transport ops (``tests/test_lap_opcheck.py:25,56-73``,
``tests/test_transport_opcheck.py:11-74``): the schema check runs the op and
verifies that no input is mutated and that the outputs match the declared
aliasing; the fake-tensor check runs the registered fake on fake inputs and
requires the same output shapes, dtypes, strides and devices as the real
kernel.  Here every op runs on ROCm tensors, so the kernels checked are the
gfx950 ones: the JV ops of ``csrc/torch_ops.cpp`` (the K <= 64 kernel and the
large-K kernel, square and rectangular, float32 and float64 input) and the
transport custom ops' ``"cuda"`` kernels (the two-sweep step at the
reference's shapes and the one-read fused step at 256 columns).
"""

from __future__ import annotations

import pytest
import torch

import torchmatch_amd  # noqa: F401

pytestmark = pytest.mark.gpu

_UTILS = ("test_schema", "test_faketensor")

JV_OPS = ["jonker_dense_batch", "jonker_compact_batch", "jonker_dense_batch_unpacked",
          "jonker_compact_batch_unpacked"]


def _rand(*shape, seed=0, dtype=torch.float32):
    return torch.rand(*shape, generator=torch.Generator().manual_seed(seed), dtype=dtype)


@pytest.mark.parametrize("op_name", JV_OPS)
@pytest.mark.parametrize("shape", [(4, 16, 16), (3, 20, 33), (2, 100, 130)],
                         ids=["4x16x16", "3x20x33", "2x100x130"])
def test_jv_ops_opcheck(op_name, shape, device):
    cost = _rand(*shape).to(device)
    print(f"opcheck assignment::{op_name} {tuple(shape)}", flush=True)
    torch.library.opcheck(getattr(torch.ops.assignment, op_name), (cost,), test_utils=_UTILS)


@pytest.mark.parametrize("op_name", ["jonker_dense_batch", "jonker_dense_batch_unpacked"])
def test_jv_ops_opcheck_float64_and_inf(op_name, device):
    cost = _rand(4, 16, 16, seed=1, dtype=torch.float64)
    cost[1, 3, :8] = float("inf")
    print(f"opcheck assignment::{op_name} float64 with +inf", flush=True)
    torch.library.opcheck(getattr(torch.ops.assignment, op_name), (cost.to(device),),
                          test_utils=_UTILS)


def _marginals(shape, device):
    b, n, m = shape
    a = torch.full((b, n), 1.0 / n, dtype=torch.float32, device=device)
    c = torch.full((b, m), 1.0 / m, dtype=torch.float32, device=device)
    return a, c


SK_SHAPES = [(2, 3, 3), (1, 3, 5), (2, 64, 256)]


@pytest.mark.parametrize("shape", SK_SHAPES, ids=[f"{b}x{n}x{m}" for b, n, m in SK_SHAPES])
def test_log_sinkhorn_opcheck(shape, device):
    cost = _rand(*shape, seed=2).to(device)
    a, b = _marginals(shape, device)
    print(f"opcheck transport::log_sinkhorn {shape}", flush=True)
    torch.library.opcheck(torch.ops.transport.log_sinkhorn, (cost, 0.1, 50, a, b),
                          kwargs={"mask": None, "scaling": None}, test_utils=_UTILS)


@pytest.mark.parametrize("shape", SK_SHAPES, ids=[f"{b}x{n}x{m}" for b, n, m in SK_SHAPES])
def test_unbalanced_sinkhorn_opcheck(shape, device):
    cost = _rand(*shape, seed=3).to(device)
    a, b = _marginals(shape, device)
    print(f"opcheck transport::unbalanced_sinkhorn {shape}", flush=True)
    torch.library.opcheck(torch.ops.transport.unbalanced_sinkhorn, (cost, 0.1, 30, 1.0, a, b),
                          kwargs={"mask": None, "scaling": None}, test_utils=_UTILS)


@pytest.mark.parametrize("shape", SK_SHAPES, ids=[f"{b}x{n}x{m}" for b, n, m in SK_SHAPES])
def test_sinkhorn_divergence_opcheck(shape, device):
    cost = _rand(*shape, seed=4).to(device)
    a, b = _marginals(shape, device)
    print(f"opcheck transport::sinkhorn_divergence {shape}", flush=True)
    torch.library.opcheck(torch.ops.transport.sinkhorn_divergence, (cost, 0.1, 30, a, b),
                          kwargs={"mask": None, "scaling": None}, test_utils=_UTILS)


def test_sinkhorn_opcheck_with_mask_and_scaling(device):
    shape = (2, 40, 256)
    cost = _rand(*shape, seed=5).to(device)
    a, b = _marginals(shape, device)
    mask = (_rand(*shape, seed=6) > 0.2).to(device)
    print("opcheck transport::log_sinkhorn with mask and scaling", flush=True)
    torch.library.opcheck(torch.ops.transport.log_sinkhorn, (cost, 0.05, 40, a, b),
                          kwargs={"mask": mask, "scaling": 0.7}, test_utils=_UTILS)
    torch.library.opcheck(torch.ops.transport.unbalanced_sinkhorn,
                          (cost, 0.05, 40, 0.5, a, b),
                          kwargs={"mask": mask, "scaling": None}, test_utils=_UTILS)
