"""tm_jv_dense_batch_f32_noalloc: the JV entry point that allocates nothing.

Its workspace is a fixed device array inside the library.  Calls in a row
through the C ABI, each on a smaller or differently shaped input than the one
before (the fused K <= 64 path, rectangular and +inf-masked inputs, the
statistics-pass path with K > 64 and with B > 2048, then the fused path again),
each compared bit for bit with tm_jv_dense_batch_f32 run on a workspace the
test allocates; the status words must agree too.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import torchmatch_amd  # noqa: F401
from torchmatch_amd import _native
import workloads

pytestmark = pytest.mark.gpu


def _vp(t: torch.Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr())


def _with_workspace(lib, cost, stream):
    B, N, M = cost.shape
    out = torch.full((B, N), -7, dtype=torch.int64, device=cost.device)
    nbytes = lib.tm_jv_workspace_bytes(B, N, M)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=cost.device)
    status = torch.zeros(2, dtype=torch.int32, device=cost.device)
    rc = lib.tm_jv_dense_batch_f32(_vp(cost), B, N, M, _vp(out), _vp(ws), nbytes, _vp(status),
                                   stream)
    assert rc == _native.TM_OK
    code = lib.tm_jv_check_status(_vp(status), stream)
    return out.cpu().numpy(), status.cpu().numpy(), code


def _no_alloc(lib, cost, stream):
    B, N, M = cost.shape
    out = torch.full((B, N), -7, dtype=torch.int64, device=cost.device)
    status = torch.full((2,), 12345, dtype=torch.int32, device=cost.device)
    rc = lib.tm_jv_dense_batch_f32_noalloc(_vp(cost), B, N, M, _vp(out), _vp(status), stream)
    assert rc == _native.TM_OK
    code = lib.tm_jv_check_status(_vp(status), stream)
    return out.cpu().numpy(), status.cpu().numpy(), code


def _masked(cost, seed, p=0.1):
    g = torch.Generator().manual_seed(seed)
    cost = cost.clone()
    cost[torch.rand(cost.shape, generator=g) < p] = float("inf")
    return cost


def test_no_alloc_matches_workspace_entry(device):
    lib = _native.lib()
    assert lib.tm_jv_noalloc_scratch_bytes() >= lib.tm_jv_workspace_bytes(4096, 1024, 1024)
    stream = ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)
    # the fused path (K <= 64, B <= 2048), then the statistics-pass path with
    # the large-K kernel (K > 64) and with the K <= 64 kernel (B > 2048), then
    # the fused path again on what those left in the scratch array
    cases = [
        ("fused (512, 64, 64)", workloads.jv_uniform(512, 64, 64, seed=11)),
        ("fused (37, 23, 41) +inf", _masked(workloads.jv_uniform(37, 23, 41, seed=12), 12)),
        ("large K (4, 100, 130) +inf", _masked(workloads.jv_uniform(4, 100, 130, seed=13), 13)),
        ("large K (3, 90, 70)", workloads.jv_uniform(3, 90, 70, seed=14)),
        ("B > 2048 (2300, 16, 16) +inf", _masked(workloads.jv_uniform(2300, 16, 16, seed=15), 15)),
        ("fused (21, 30, 30) +inf", _masked(workloads.jv_uniform(21, 30, 30, seed=16), 16)),
    ]
    for label, cost in cases:
        print(f"no-alloc: {label}", flush=True)
        cost = cost.to(device)
        want, want_status, want_code = _with_workspace(lib, cost, stream)
        got, got_status, got_code = _no_alloc(lib, cost, stream)
        assert got_code == want_code == _native.TM_OK, label
        np.testing.assert_array_equal(got_status, want_status, err_msg=label)
        np.testing.assert_array_equal(got, want, err_msg=label)
