"""Parity of the gfx950 compact JV kernel with the reference CPU op
``assignment::jonker_compact_batch`` (bit-exact mappings).

The reference has no device version of this op; the CPU op runs the square
solver of jonker_compact_core.h:20-252 inside the batch driver of
ops.cpp:176-289 (sentinel, padding), and torchmatch's CPU AUTO routes square
batches there (assignment/_solve.py:75-76).  Checked against the committed
golden fixtures (the "compact" mappings, written from the reference's own
compiled header) and against the pinned C oracle (jvoc_square) on seeded
inputs: uniform, integer-tied, +inf-masked, gated-sparse, rectangular both
ways, K = 1..64 and large K up to 1024 (the second kernel), negative and
huge magnitudes (the lane-serial paths), -0.0, all-+inf problems, plus the
NaN / -inf contract and the unpacked tuple.
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch

import torchmatch_amd  # noqa: F401
from oracle import jv
from torchmatch_amd import _native
import jv_inputs
import workloads

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"


def _max_k() -> int:
    return int(_native.lib().tm_jv_compact_max_k())


def run_op(cost, device) -> np.ndarray:
    out = torch.ops.assignment.jonker_compact_batch(torch.as_tensor(cost).to(device))
    torch.cuda.synchronize()
    return out.cpu().numpy()


def _golden_cases():
    index = json.loads((GOLDEN / "jv_golden.json").read_text())
    return sorted(index.items())


@pytest.mark.parametrize(("name", "meta"), _golden_cases(), ids=[n for n, _ in _golden_cases()])
def test_golden_fixture(name, meta, device):
    b, n, m = meta["shape"]
    if max(n, m) > _max_k():
        pytest.skip(f"K={max(n, m)} beyond the compact kernel's limit {_max_k()}")
    cost = getattr(workloads, meta["generator"])(**meta["kwargs"])
    assert workloads.sha256(cost) == meta["sha256"], "input generator drifted"
    want = np.load(GOLDEN / meta["file"])["compact"].astype(np.int64)
    print(f"compact case {name} shape {tuple(cost.shape)}", flush=True)
    got = run_op(cost, device)
    mism = np.argwhere((got != want).any(axis=1)).ravel()
    assert mism.size == 0, f"{mism.size} problems differ, first {mism[:8].tolist()}"


@pytest.mark.parametrize("kind", jv_inputs.KINDS_COMPACT)
def test_random_batches_match_oracle(kind, device):
    for n, m, c in jv_inputs.compact_small_batches(kind, min(_max_k(), 64)):
        print(f"compact {kind} {c.shape}", flush=True)
        want = jv.jv_compact_batch(c)
        got = run_op(c, device)
        mism = np.argwhere((got != want).any(axis=1)).ravel()
        assert mism.size == 0, f"{kind} {c.shape}: {mism.size} problems differ"


@pytest.mark.parametrize("kind", jv_inputs.KINDS_COMPACT_LARGE)
def test_large_k_match_oracle(kind, device):
    """64 < K <= 1024: the large-K compact kernel (and its lane-serial path for
    huge magnitudes)."""
    if _max_k() <= 64:
        pytest.skip("no large-K compact kernel in this build")
    for n, m, c in jv_inputs.compact_large_batches(kind):
        print(f"compact large {kind} {c.shape}", flush=True)
        want = jv.jv_compact_batch(c)
        got = run_op(c, device)
        mism = np.argwhere((got != want).any(axis=1)).ravel()
        assert mism.size == 0, f"{kind} {c.shape}: {mism.size} problems differ"


@pytest.mark.parametrize("kind", jv_inputs.KINDS_XL)
def test_xl_k_match_oracle(kind, device):
    """1024 < K <= 2048: the compact solver on the cache-less 32-chunk
    instantiation."""
    assert _max_k() >= 2048
    for n, m, c in jv_inputs.xl_batches(kind):
        print(f"compact xl {kind} {c.shape}", flush=True)
        want = jv.jv_compact_batch(c)
        got = run_op(c, device)
        mism = np.argwhere((got != want).any(axis=1)).ravel()
        assert mism.size == 0, f"{kind} {c.shape}: {mism.size} problems differ"


def test_every_k_up_to_limit(device):
    rng = np.random.default_rng(31)
    for k in range(1, min(_max_k(), 64) + 1):
        c = rng.integers(0, 4, (16, k, k)).astype(np.float32)
        np.testing.assert_array_equal(run_op(c, device), jv.jv_compact_batch(c))


def test_all_inf_and_known_answers(device):
    inf = np.inf
    c = np.array([[[1.0, inf], [inf, 1.0]], [[2.0, inf], [inf, 3.0]]], dtype=np.float32)
    assert run_op(c, device).tolist() == [[0, 1], [0, 1]]
    c = np.full((4, 6, 6), np.inf, np.float32)
    np.testing.assert_array_equal(run_op(c, device), jv.jv_compact_batch(c))
    assert (run_op(np.zeros((3, 4, 0), np.float32), device) == -1).all()


def test_nan_and_neg_inf_raise(device):
    c = torch.rand(4, 8, 8)
    c[2, 3, 3] = float("nan")
    with pytest.raises(RuntimeError, match="NaN"):
        torch.ops.assignment.jonker_compact_batch(c.to(device))
    c[2, 3, 3] = -float("inf")
    with pytest.raises(RuntimeError, match="-inf"):
        torch.ops.assignment.jonker_compact_batch(c.to(device))


def test_unpacked_tuple_matches_cpu_format(device):
    c = workloads.integer_tied(32, 20, 30, seed=4, hi=3)
    got = torch.ops.assignment.jonker_compact_batch_unpacked(c.to(device))
    want = jv.unpack_packed(jv.jv_compact_batch(c.numpy()), 30)
    for g, w in zip(got, want):
        np.testing.assert_array_equal(g.cpu().numpy(), w)


def test_differs_from_dense_on_ties(device):
    """The two ops must not collapse into one: on tied costs their mappings
    differ exactly where the CPU ops' do."""
    c = workloads.integer_tied(64, 32, 32, seed=8, hi=3)
    compact = run_op(c, device)
    dense = torch.ops.assignment.jonker_dense_batch(c.to(device)).cpu().numpy()
    np.testing.assert_array_equal(compact, jv.jv_compact_batch(c.numpy()))
    np.testing.assert_array_equal(dense, jv.jv_dense_batch(c.numpy()))
    assert (compact != dense).any(axis=1).sum() > 32


def test_edge_contracts(device):
    """Empty shapes, float64 (solved in float32, as the device JV op does),
    non-contiguous input and the K limit, as for the dense op."""
    for shape in [(0, 4, 4), (3, 0, 4), (3, 4, 0)]:
        out = torch.ops.assignment.jonker_compact_batch(torch.empty(shape, device=device))
        assert out.shape == shape[:2] and (out == -1).all()
    c64 = torch.rand(32, 20, 20, dtype=torch.float64)
    want = jv.jv_compact_batch(c64.to(torch.float32).numpy())
    np.testing.assert_array_equal(run_op(c64, device), want)
    with pytest.raises(RuntimeError, match="contiguous"):
        torch.ops.assignment.jonker_compact_batch(
            torch.rand(4, 8, 8, device=device).transpose(1, 2))
    k = _max_k() + 1
    with pytest.raises(RuntimeError, match="K"):
        torch.ops.assignment.jonker_compact_batch(torch.rand(1, k, k, device=device))


def test_c_abi_direct(device):
    """The compact entry through the C ABI with raw device pointers."""
    lib = _native.lib()
    cost = workloads.integer_tied(128, 48, 64, seed=12, hi=3)
    dc = cost.to(device)
    out = torch.empty(128, 48, dtype=torch.int64, device=device)
    ws_bytes = lib.tm_jv_workspace_bytes(128, 48, 64)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=device)
    status = torch.zeros(2, dtype=torch.int32, device=device)
    stream = torch.cuda.current_stream(device).cuda_stream
    rc = lib.tm_jv_compact_batch_f32(dc.data_ptr(), 128, 48, 64, out.data_ptr(), ws.data_ptr(),
                                     ws_bytes, status.data_ptr(), stream)
    assert rc == _native.TM_OK
    assert lib.tm_jv_check_status(status.data_ptr(), stream) == _native.TM_OK
    np.testing.assert_array_equal(out.cpu().numpy(), jv.jv_compact_batch(cost.numpy()))
    rc = lib.tm_jv_compact_batch_f32(dc.data_ptr(), 128, 48, 64, out.data_ptr(),
                                     ws.data_ptr(), 8, status.data_ptr(), stream)
    assert rc == _native.TM_ERR_WORKSPACE
