"""The K <= 64 launch without a statistics pass (B <= 2048).

The solve launch takes each tile's own statistics and solves every problem
without +inf; problems holding +inf wait for the finishing launch, which folds
the per-problem records into the batch statistics (the reference's
batch-global sentinel (max finite + 1) * (K + 1), ops.cpp:67-93) and the
status words.  These tests hold that split to the oracle:

* mixed batches (some problems with +inf, some without), dense and compact,
  on both sides of the B = 2048 limit (above it the statistics pass runs);
* a workspace full of garbage (the contract says "any contents");
* NaN / -inf anywhere: the error code, and -1 in every output;
* the status flags of the whole batch, and the guard word cleared between
  calls;
* TM_JV_FLAG_DONE: set by batches whose problems are all solved in the first
  launch, never by batches that defer a problem or take the statistics pass;
* the synchronous entry points (tm_jv_*_batch_f32_sync), which fold the
  problems' summaries on the host: the same mappings and error codes, -1 in
  every output on NaN / -inf, and the replay count.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import torchmatch_amd  # noqa: F401
from oracle import jv
from torchmatch_amd import _native

pytestmark = pytest.mark.gpu

FLAG_POS_INF = 4
FLAG_ANY_FINITE = 8
FLAG_NEG_ZERO = 16
FLAG_DONE = 0x80000000


def _abi(cost: torch.Tensor, device, compact: bool = False, garbage: bool = True):
    """(rc of the launch, status code, status words, mapping) through the C ABI."""
    lib = _native.lib()
    c = cost.to(device).contiguous()
    B, N, M = c.shape
    out = torch.full((B, N), 12345, dtype=torch.int64, device=device)
    nbytes = lib.tm_jv_workspace_bytes(B, N, M)
    ws = torch.full((nbytes,), 0xA5 if garbage else 0, dtype=torch.uint8, device=device)
    status = torch.full((2,), 7, dtype=torch.int32, device=device)
    stream = ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)
    fn = lib.tm_jv_compact_batch_f32 if compact else lib.tm_jv_dense_batch_f32
    rc = fn(ctypes.c_void_p(c.data_ptr()), B, N, M, ctypes.c_void_p(out.data_ptr()),
            ctypes.c_void_p(ws.data_ptr()), nbytes, ctypes.c_void_p(status.data_ptr()), stream)
    code = lib.tm_jv_check_status(ctypes.c_void_p(status.data_ptr()), stream)
    return rc, code, status.cpu().numpy().astype(np.uint32), out.cpu().numpy()


def _mixed(B: int, N: int, M: int, seed: int, frac_inf: float = 0.5) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    c = torch.rand(B, N, M, generator=g)
    masked = torch.rand(B, generator=g) < frac_inf
    holes = torch.rand(B, N, M, generator=g) < 0.15
    c[masked.view(B, 1, 1) & holes] = float("inf")
    return c


@pytest.mark.parametrize("compact", [False, True])
@pytest.mark.parametrize(("B", "N", "M"), [(300, 48, 48), (257, 64, 64), (200, 30, 41),
                                            (2048, 16, 16), (2049, 16, 16)])
def test_mixed_inf_batches_match_oracle(B, N, M, compact, device):
    cost = _mixed(B, N, M, seed=B + N + M)
    rc, code, st, got = _abi(cost, device, compact=compact)
    assert rc == _native.TM_OK and code == _native.TM_OK
    want = (jv.jv_compact_batch if compact else jv.jv_dense_batch)(cost.numpy())
    bad = np.nonzero((got != want).any(axis=1))[0]
    print(f"mixed {(B, N, M)} compact={compact}: {len(bad)} problems differ", flush=True)
    assert len(bad) == 0
    assert st[0] & FLAG_POS_INF and st[0] & FLAG_ANY_FINITE and st[1] == 0
    assert not st[0] & FLAG_DONE  # +inf problems were solved by the finishing launch


@pytest.mark.parametrize("B", [64, 2049])
@pytest.mark.parametrize(("value", "err"), [(float("nan"), _native.TM_ERR_NAN),
                                            (float("-inf"), _native.TM_ERR_NEG_INF)])
def test_nan_and_neg_inf_fill_every_output(B, value, err, device):
    cost = _mixed(B, 64 if B < 2048 else 8, 64 if B < 2048 else 8, seed=3, frac_inf=0.3)
    cost[B // 3, 2, 5] = value
    rc, code, _, got = _abi(cost, device)
    assert rc == _native.TM_OK
    assert code == err
    assert (got == -1).all()


def test_status_flags_and_guard_cleared(device):
    cost = torch.rand(128, 64, 64, generator=torch.Generator().manual_seed(9))
    cost[5, 0, 0] = -0.0
    rc, code, st, got = _abi(cost, device)
    assert rc == _native.TM_OK and code == _native.TM_OK
    assert st[0] == FLAG_DONE | FLAG_ANY_FINITE | FLAG_NEG_ZERO and st[1] == 0
    assert (got == jv.jv_dense_batch(cost.numpy())).all()
    # a clean call after a batch with +inf reports no +inf
    _abi(_mixed(64, 64, 64, seed=4), device)
    rc, code, st, _ = _abi(torch.rand(64, 64, 64), device)
    assert rc == _native.TM_OK and code == _native.TM_OK
    assert st[0] == FLAG_DONE | FLAG_ANY_FINITE and st[1] == 0
    # the statistics-pass path (B > 2048) never sets the done bit
    rc, code, st, _ = _abi(torch.rand(2049, 8, 8), device)
    assert rc == _native.TM_OK and code == _native.TM_OK
    assert st[0] == FLAG_ANY_FINITE and st[1] == 0


def test_all_inf_problem_uses_batch_sentinel(device):
    """A problem that is +inf everywhere takes the sentinel from the other
    problems' finite values (ops.cpp:67-93), like the reference."""
    cost = torch.rand(40, 20, 20, generator=torch.Generator().manual_seed(1)) * 5
    cost[7] = float("inf")
    cost[8, :, 3] = float("inf")
    rc, code, _, got = _abi(cost, device)
    assert rc == _native.TM_OK and code == _native.TM_OK
    assert (got == jv.jv_dense_batch(cost.numpy())).all()


def _sync(cost: torch.Tensor, device, compact: bool = False):
    """(status code, replays, mapping) through the synchronous C ABI."""
    lib = _native.lib()
    c = cost.to(device).contiguous()
    B, N, M = c.shape
    out = torch.full((B, N), 12345, dtype=torch.int64, device=device)
    nbytes = lib.tm_jv_workspace_bytes(B, N, M)
    ws = torch.full((nbytes,), 0xA5, dtype=torch.uint8, device=device)
    stream = ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)
    fn = lib.tm_jv_compact_batch_f32_sync if compact else lib.tm_jv_dense_batch_f32_sync
    replays = ctypes.c_uint32(77)
    code = fn(ctypes.c_void_p(c.data_ptr()), B, N, M, ctypes.c_void_p(out.data_ptr()),
              ctypes.c_void_p(ws.data_ptr()), nbytes, ctypes.byref(replays), stream)
    return code, replays.value, out.cpu().numpy()


@pytest.mark.parametrize("compact", [False, True])
@pytest.mark.parametrize(("B", "N", "M", "frac_inf"), [(300, 64, 64, 0.0), (300, 48, 48, 0.5),
                                                       (200, 30, 41, 0.0), (2049, 16, 16, 0.3)])
def test_sync_entry_matches_oracle(B, N, M, frac_inf, compact, device):
    cost = _mixed(B, N, M, seed=7 * B + N, frac_inf=frac_inf)
    code, replays, got = _sync(cost, device, compact=compact)
    assert code == _native.TM_OK
    want = (jv.jv_compact_batch if compact else jv.jv_dense_batch)(cost.numpy())
    assert (got == want).all()
    assert replays <= B


@pytest.mark.parametrize("compact", [False, True])
def test_small_k_after_large_tiles(compact, device):
    """Tiles with K < 64 are stored up to the next 16-row boundary (0 past
    K), and the column build and the certificate stop there.  Regression
    test for rows left unset: stale LDS words from the 64 x 64 tiles of large
    costs solved just before, on as many workgroups, would enter the
    certificate's cost scale (tau = 2^-20 max |c|) and send the square
    problems to the exact replay: the same mappings, but counted."""
    g = torch.Generator().manual_seed(31)
    big = torch.rand(1024, 64, 64, generator=g) * 1e6
    for n, m in [(5, 5), (17, 17), (20, 20), (33, 33), (47, 47), (30, 41)]:
        cost = torch.rand(1024, n, m, generator=g)
        print(f"large tiles, then {tuple(cost.shape)} compact={compact}", flush=True)
        assert _sync(big, device, compact=compact)[0] == _native.TM_OK
        code, replays, got = _sync(cost, device, compact=compact)
        assert code == _native.TM_OK
        want = (jv.jv_compact_batch if compact else jv.jv_dense_batch)(cost.numpy())
        assert (got == want).all()
        # uniform costs: near-ties within tau are rare (a few per 10^4 problems)
        assert replays <= 8, f"{replays} replays on {tuple(cost.shape)}"


def test_sync_replay_count_and_errors(device):
    # integer ties: every square problem fails the certificate and replays
    g = torch.Generator().manual_seed(5)
    cost = torch.randint(0, 4, (256, 32, 32), generator=g).float()
    code, replays, got = _sync(cost, device)
    assert code == _native.TM_OK and replays >= 250
    assert (got == jv.jv_dense_batch(cost.numpy())).all()
    for value, err in ((float("nan"), _native.TM_ERR_NAN), (float("-inf"), _native.TM_ERR_NEG_INF)):
        bad = torch.rand(128, 64, 64, generator=g)
        bad[77, 3, 9] = value
        code, _, got = _sync(bad, device)
        assert code == err
        assert (got == -1).all()
    # a clean call right after an error call
    clean = torch.rand(128, 64, 64, generator=g)
    code, _, got = _sync(clean, device)
    assert code == _native.TM_OK
    assert (got == jv.jv_dense_batch(clean.numpy())).all()
