"""tm_jv_dense_batch_f32_noalloc: the JV entry point that allocates nothing.

Its workspace is a fixed device array inside the library.  Two calls in a
row through the C ABI, the second on a smaller (and rectangular, +inf-masked)
input, each compared bit for bit with tm_jv_dense_batch_f32 run on a
workspace the test allocates; the status words must agree too.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import torchmatch_amd  # noqa: F401
from torchmatch_amd import _native, workloads

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


def test_no_alloc_matches_workspace_entry(device):
    lib = _native.lib()
    assert lib.tm_jv_noalloc_scratch_bytes() >= lib.tm_jv_workspace_bytes(4096, 1024, 1024)
    stream = ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)
    big = workloads.jv_uniform(512, 64, 64, seed=11).to(device)
    small = workloads.jv_uniform(37, 23, 41, seed=12)
    small[small < 0.1] = float("inf")
    small = small.to(device)
    print("no-alloc: (512, 64, 64) then (37, 23, 41) with +inf", flush=True)
    for cost in (big, small):
        want, want_status, want_code = _with_workspace(lib, cost, stream)
        got, got_status, got_code = _no_alloc(lib, cost, stream)
        assert got_code == want_code == _native.TM_OK
        np.testing.assert_array_equal(got_status, want_status)
        np.testing.assert_array_equal(got, want)
