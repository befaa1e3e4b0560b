"""Re-entrancy of the Sinkhorn C ABI (the reference ops keep no global mutable
state, so callers may run them from several threads at once).

The fused step splits a batch into groups on the caller's stream and on side
streams the library owns, one set per device.  Two host threads call
``tm_sinkhorn_f32`` through ctypes (which releases the GIL for the call), each
on its own torch stream with its own problem and workspace, many times in a
row, so their fork / launch / join segments overlap in time.  Every result
must equal, bit for bit, the same solve run alone with one group
(TORCHMATCH_AMD_SINKHORN_GROUPS=1: every launch on the caller's stream).
"""

from __future__ import annotations

import ctypes
import threading

import pytest
import torch

import torchmatch_amd  # noqa: F401
from torchmatch_amd import _native
import workloads

pytestmark = pytest.mark.gpu


def _ptr(t: torch.Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr())


class _Problem:
    def __init__(self, B, N, M, eps, n_iter, rho, seed, device):
        self.dims = (B, N, M)
        self.cost = workloads.sinkhorn_points(B, N, M, 8, seed=seed).to(device)
        self.a = workloads.dirichlet(B, N, 1.0, seed=seed + 1).to(device)
        self.b = workloads.dirichlet(B, M, 1.3 if rho > 0 else 1.0, seed=seed + 2).to(device)
        self.sched = (ctypes.c_double * n_iter)(*([eps] * n_iter))
        self.n_iter, self.rho = n_iter, rho
        nbytes = _native.lib().tm_sinkhorn_workspace_bytes(B, N, M)
        self.ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
        self.plan = torch.empty(B, N, M, device=device)
        self.log_u = torch.empty(B, N, device=device)
        self.log_v = torch.empty(B, M, device=device)

    def run(self, stream: torch.cuda.Stream) -> int:
        B, N, M = self.dims
        return _native.lib().tm_sinkhorn_f32(
            _ptr(self.cost), _ptr(self.a), _ptr(self.b), B, N, M, self.sched, self.n_iter,
            self.rho, _ptr(self.plan), _ptr(self.log_u), _ptr(self.log_v), _ptr(self.ws),
            self.ws.numel(), ctypes.c_void_p(stream.cuda_stream))

    def result(self, stream: torch.cuda.Stream):
        """Copies of the outputs, made on ``stream`` after the solve and
        finished before the next solve on it rewrites them."""
        with torch.cuda.stream(stream):
            out = self.plan.clone(), self.log_u.clone(), self.log_v.clone()
        stream.synchronize()
        return out


def test_two_threads_two_streams_match_serial(device, monkeypatch):
    probs = [
        _Problem(4, 300, 1024, 0.05, 40, 0.0, seed=51, device=device),
        _Problem(3, 200, 2048, 0.02, 40, 1.0, seed=61, device=device),
    ]
    torch.cuda.synchronize()
    # alone, one group on one stream
    monkeypatch.setenv("TORCHMATCH_AMD_SINKHORN_GROUPS", "1")
    serial = []
    for p in probs:
        s = torch.cuda.Stream(device)
        assert p.run(s) == _native.TM_OK
        serial.append(p.result(s))
    monkeypatch.delenv("TORCHMATCH_AMD_SINKHORN_GROUPS")

    reps = 12
    errors: list[str] = []
    results: list[list] = [[], []]
    start = threading.Barrier(2)

    def worker(k: int) -> None:
        p = probs[k]
        s = torch.cuda.Stream(device)
        start.wait()
        for _ in range(reps):
            rc = p.run(s)
            if rc != _native.TM_OK:
                errors.append(f"thread {k}: rc {rc}")
                return
            results[k].append(p.result(s))

    threads = [threading.Thread(target=worker, args=(k,)) for k in range(2)]
    print("two threads, two streams, default batch groups", flush=True)
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=100)
    assert not any(t.is_alive() for t in threads), "a worker thread did not finish"
    assert not errors, errors
    for k in range(2):
        assert len(results[k]) == reps
        for plan, lu, lv in results[k]:
            assert torch.equal(plan, serial[k][0])
            assert torch.equal(lu, serial[k][1])
            assert torch.equal(lv, serial[k][2])
