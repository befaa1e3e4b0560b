"""The certified shortest-path solve of the K <= 64 JV kernel and its fallback.

Square tiles of finite costs are first solved without the reference's
augmenting row reduction; the kernel keeps that result only when a float64
certificate proves it is the unique optimum by a margin of 2^-20 of the
largest |cost|, and otherwise solves the problem again by the exact replay of
the reference's order.  Checked here:

* the mappings equal the oracle (bit-exact) with the certified path on and
  off (TORCHMATCH_AMD_JV_CERTIFY=0), on eight C2 batches and on the
  reference's compact solver;
* the replay count the kernel reports (tm_jv_read_replays): near zero on
  uniform costs, every problem on integer-tied costs, and exactly the
  problems into which a tie or a near-tie (gap below the margin) was planted.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import torchmatch_amd  # noqa: F401
from oracle import jv
from torchmatch_amd import _native
import workloads

pytestmark = pytest.mark.gpu


def _solve_abi(cost: torch.Tensor, device, compact: bool = False):
    """(mapping, replays) through the C ABI."""
    lib = _native.lib()
    c = cost.to(device).contiguous()
    B, N, M = c.shape
    out = torch.empty(B, N, dtype=torch.int64, device=device)
    nbytes = lib.tm_jv_workspace_bytes(B, N, M)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
    status = torch.zeros(2, dtype=torch.int32, device=device)
    stream = ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)
    fn = lib.tm_jv_compact_batch_f32 if compact else lib.tm_jv_dense_batch_f32
    rc = fn(ctypes.c_void_p(c.data_ptr()), B, N, M, ctypes.c_void_p(out.data_ptr()),
            ctypes.c_void_p(ws.data_ptr()), nbytes, ctypes.c_void_p(status.data_ptr()), stream)
    assert rc == _native.TM_OK
    assert lib.tm_jv_check_status(ctypes.c_void_p(status.data_ptr()), stream) == _native.TM_OK
    count = ctypes.c_uint32(0)
    assert lib.tm_jv_read_replays(ctypes.c_void_p(ws.data_ptr()), ctypes.byref(count),
                                  stream) == _native.TM_OK
    return out.cpu().numpy(), count.value


@pytest.mark.parametrize("certify", ["1", "0"])
def test_c2_batches_bit_exact_both_paths(certify, device, monkeypatch):
    monkeypatch.setenv("TORCHMATCH_AMD_JV_CERTIFY", certify)
    total = 0
    for seed in range(8):
        cost = workloads.jv_uniform(1024, 64, 64, seed=100 + seed)
        want = jv.jv_dense_batch(cost.numpy())
        got, replays = _solve_abi(cost, device)
        print(f"certify={certify} seed {100 + seed}: replays {replays}", flush=True)
        np.testing.assert_array_equal(got, want)
        if certify == "0":
            assert replays == 0   # the certified path did not run
        total += replays
    if certify == "1":
        assert total <= 40        # about 1 in 3,000 problems on uniform costs


@pytest.mark.parametrize("certify", ["1", "0"])
def test_compact_bit_exact_both_paths(certify, device, monkeypatch):
    monkeypatch.setenv("TORCHMATCH_AMD_JV_CERTIFY", certify)
    cost = workloads.jv_uniform(1024, 64, 64, seed=7)
    want = jv.jv_compact_batch(cost.numpy())
    got, replays = _solve_abi(cost, device, compact=True)
    print(f"compact certify={certify}: replays {replays}", flush=True)
    np.testing.assert_array_equal(got, want)


def test_integer_ties_all_replay(device):
    cost = workloads.integer_tied(256, 64, 64, seed=1)
    got, replays = _solve_abi(cost, device)
    print(f"integer-tied replays {replays} / 256", flush=True)
    np.testing.assert_array_equal(got, jv.jv_dense_batch(cost.numpy()))
    assert replays >= 250
    got_c, _ = _solve_abi(cost, device, compact=True)
    np.testing.assert_array_equal(got_c, jv.jv_compact_batch(cost.numpy()))


@pytest.mark.parametrize("gap", [0.0, 2e-7, 1e-3])
def test_planted_swap_gap(gap, device):
    """Rows 3 and 17 may only take columns 10 and 40 (every other entry of
    the two rows is 4, far above the rest's [0.25, 0.75)); one way costs
    0.25 + 0.25, the other `gap` more.  The optimum is then unique for
    gap > 0 with the swap `gap` behind it.  A tie (0) and a near-tie (2e-7,
    below the margin 2^-20 * 4 ~ 3.8e-6) must take the exact replay; a clear
    gap (1e-3) must not."""
    rng = np.random.default_rng(5)
    B, n = 64, 64
    c = rng.random((B, n, n), dtype=np.float32) * np.float32(0.5) + np.float32(0.25)
    i, k, a, b = 3, 17, 10, 40
    c[:, i, :] = 4.0
    c[:, k, :] = 4.0
    c[:, i, a] = 0.25
    c[:, k, b] = 0.25
    c[:, k, a] = 0.25
    c[:, i, b] = np.float32(0.25 + gap)
    got, replays = _solve_abi(torch.from_numpy(c), device)
    print(f"planted gap {gap}: replays {replays} / {B}", flush=True)
    np.testing.assert_array_equal(got, jv.jv_dense_batch(c))
    if gap < 1e-6:
        assert replays == B
    else:
        assert replays <= 2
