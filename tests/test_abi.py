"""The C ABI library loads, exports every declared symbol, and the torch
layer registers the reference's schemas -- no GPU needed."""

from __future__ import annotations

import re
from pathlib import Path

import pytest
import torch

import torchmatch_amd
from torchmatch_amd import _native
from torchmatch_amd._loader import CABI_SO, OPS_SO

HEADER = Path(__file__).resolve().parents[1] / "include" / "torchmatch_amd.h"


def _declared_functions() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tm_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_bound_functions():
    declared = _declared_functions()
    assert declared == sorted(_native.SIGNATURES), declared


@pytest.mark.parametrize("name", _declared_functions())
def test_library_exports_symbol(name):
    assert CABI_SO.exists() and OPS_SO.exists()
    assert hasattr(_native.lib(), name)


def test_workspace_queries():
    lib = _native.lib()
    assert lib.tm_jv_max_k() >= 64
    assert lib.tm_jv_workspace_bytes(1024, 64, 64) >= 256
    # the prefill size: equal for K <= 64, larger for K > 64 (C3: ~3.7 MB,
    # of which 3.1 MB are the 16-slot row caches: 6 bytes per slot)
    assert lib.tm_jv_workspace_bytes_prefill(1024, 64, 64) == lib.tm_jv_workspace_bytes(1024, 64, 64)
    c3 = lib.tm_jv_workspace_bytes_prefill(64, 512, 768)
    assert lib.tm_jv_workspace_bytes(64, 512, 768) + 64 * 512 * 16 * 6 < c3 < 4 << 20
    small = lib.tm_sinkhorn_workspace_bytes(2, 8, 8)
    big = lib.tm_sinkhorn_workspace_bytes(16, 2048, 2048)
    assert big > 16 * 2048 * 2048 * 4 > small


def test_invalid_arguments_rejected_without_gpu_work():
    lib = _native.lib()
    # negative sizes are rejected before any launch
    assert lib.tm_jv_dense_batch_f32(None, -1, 4, 4, None, None, 0, None, None) == \
        _native.TM_ERR_INVALID_ARGUMENT
    # empty batches launch nothing
    assert lib.tm_jv_dense_batch_f32(None, 0, 4, 4, None, None, 0, None, None) == _native.TM_OK
    assert lib.tm_sinkhorn_f32(None, None, None, 1, 1, 1, None, 0, 0.0, None, None, None,
                               None, 0, None) == _native.TM_ERR_INVALID_ARGUMENT


def test_schemas_match_reference():
    assert str(torch.ops.assignment.jonker_dense_batch.default._schema) == \
        "assignment::jonker_dense_batch(Tensor costs) -> Tensor"
    assert str(torch.ops.assignment.jonker_dense_batch_unpacked.default._schema) == (
        "assignment::jonker_dense_batch_unpacked(Tensor costs) -> "
        "(Tensor, Tensor, Tensor, Tensor)"
    )
    assert str(torch.ops.assignment.jonker_compact_batch.default._schema) == \
        "assignment::jonker_compact_batch(Tensor costs) -> Tensor"
    assert str(torch.ops.assignment.jonker_compact_batch_unpacked.default._schema) == (
        "assignment::jonker_compact_batch_unpacked(Tensor costs) -> "
        "(Tensor, Tensor, Tensor, Tensor)"
    )
    assert str(torch.ops.transport.log_sinkhorn.default._schema) == (
        "transport::log_sinkhorn(Tensor cost, float eps, SymInt n_iter, Tensor a, Tensor b, "
        "Tensor? mask=None, float? scaling=None) -> Tensor"
    )
    assert str(torch.ops.transport.unbalanced_sinkhorn.default._schema) == (
        "transport::unbalanced_sinkhorn(Tensor cost, float eps, SymInt n_iter, float rho, "
        "Tensor a, Tensor b, Tensor? mask=None, float? scaling=None) -> Tensor"
    )
    assert str(torch.ops.transport.sinkhorn_divergence.default._schema) == (
        "transport::sinkhorn_divergence(Tensor cost, float eps, SymInt n_iter, Tensor a, "
        "Tensor b, Tensor? mask=None, float? scaling=None, Tensor? cost_aa=None, "
        "Tensor? cost_bb=None) -> Tensor"
    )


def test_ops_modules_are_the_registered_ops():
    """The reference's import paths for the op handles
    (assignment/ops.py:17-28, transport/matrix/ops.py:8-10) resolve to the
    ops this package registers, under the reference's names."""
    from torchmatch_amd.assignment import ops as aops
    from torchmatch_amd.transport.matrix import ops as tops

    assert sorted(aops.__all__) == ["jonker_compact_batch", "jonker_compact_batch_unpacked",
                                    "jonker_dense_batch", "jonker_dense_batch_unpacked"]
    for name in aops.__all__:
        assert getattr(aops, name) is getattr(torch.ops.assignment, name)
    assert sorted(tops.__all__) == ["log_sinkhorn", "sinkhorn_divergence", "unbalanced_sinkhorn"]
    for name in tops.__all__:
        assert getattr(tops, name) is getattr(torch.ops.transport, name)


def test_no_host_fallback():
    """CPU tensors are refused loudly: the package has no host path."""
    with pytest.raises(NotImplementedError):
        torch.ops.assignment.jonker_dense_batch(torch.rand(2, 3, 3))
    with pytest.raises(NotImplementedError):
        torch.ops.assignment.jonker_compact_batch(torch.rand(2, 3, 3))
    with pytest.raises(ValueError, match="ROCm"):
        torchmatch_amd.assignment.solve(torch.rand(2, 3, 3))
    with pytest.raises(NotImplementedError):
        torch.ops.transport.log_sinkhorn(
            torch.rand(1, 3, 3), 0.1, 5, torch.full((1, 3), 1 / 3), torch.full((1, 3), 1 / 3)
        )


def test_fake_kernels():
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        c = torch.empty(5, 7, 9)
        out = torch.ops.assignment.jonker_dense_batch(c)
        assert out.shape == (5, 7) and out.dtype == torch.long
        shapes = [t.shape for t in torch.ops.assignment.jonker_dense_batch_unpacked(c)]
        assert shapes == [(5, 7, 2), (5, 7), (5, 9), (5,)]
        out = torch.ops.assignment.jonker_compact_batch(c)
        assert out.shape == (5, 7) and out.dtype == torch.long
        shapes = [t.shape for t in torch.ops.assignment.jonker_compact_batch_unpacked(c)]
        assert shapes == [(5, 7, 2), (5, 7), (5, 9), (5,)]
        plan = torch.ops.transport.log_sinkhorn(c, 0.1, 3, torch.empty(5, 7), torch.empty(5, 9))
        assert plan.shape == (5, 7, 9)
        plan = torch.ops.transport.unbalanced_sinkhorn(
            c, 0.1, 3, 1.0, torch.empty(5, 7), torch.empty(5, 9)
        )
        assert plan.shape == (5, 7, 9)
        div = torch.ops.transport.sinkhorn_divergence(c, 0.1, 3, torch.empty(5, 7),
                                                      torch.empty(5, 9))
        assert div.shape == (5,)
