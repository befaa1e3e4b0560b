"""Parity of the gfx950 JV kernel with the reference CPU op (bit-exact mappings).

Checked against the committed golden fixtures (written from the reference's
own compiled solver) and against the pinned C oracle on seeded inputs:
uniform, integer-tied, +inf-masked, gated-sparse, rectangular both ways,
K = 1..64, negative and huge magnitudes (the lane-serial path), all-+inf
problems, and the reference tests' known answers and error contracts
(test_lap_inf_mask.py, test_cudagraph_guard.py).
"""

from __future__ import annotations

import ctypes
import json
import subprocess
import sys
import textwrap
import zlib
from pathlib import Path

import numpy as np
import pytest
import torch

import torchmatch_amd
from oracle import jv
from torchmatch_amd import _native
import jv_inputs
import workloads
from torchmatch_amd.assignment import assignment_cost

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
ROOT = Path(__file__).resolve().parents[1]


def run_op(cost: torch.Tensor, device) -> np.ndarray:
    out = torch.ops.assignment.jonker_dense_batch(cost.to(device))
    torch.cuda.synchronize()
    return out.cpu().numpy()


def _golden_cases():
    index = json.loads((GOLDEN / "jv_golden.json").read_text())
    return sorted(index.items())


@pytest.mark.parametrize(("name", "meta"), _golden_cases(), ids=[n for n, _ in _golden_cases()])
def test_golden_fixture(name, meta, device):
    b, n, m = meta["shape"]
    if max(n, m) > _native.jv_max_k():
        pytest.skip(f"K={max(n, m)} beyond this build's kernel limit {_native.jv_max_k()}")
    cost = getattr(workloads, meta["generator"])(**meta["kwargs"])
    assert workloads.sha256(cost) == meta["sha256"], "input generator drifted"
    want = np.load(GOLDEN / meta["file"])["mapping"].astype(np.int64)
    print(f"case {name} shape {tuple(cost.shape)}", flush=True)
    got = run_op(cost, device)
    mism = np.argwhere((got != want).any(axis=1)).ravel()
    assert mism.size == 0, f"{mism.size} problems differ, first {mism[:8].tolist()}"


@pytest.mark.parametrize("kind", jv_inputs.KINDS_SMALL)
def test_random_batches_vs_oracle(kind, device):
    for n, m, c in jv_inputs.small_batches(kind):
        want = jv.jv_dense_batch(c)
        print(f"kind {kind} shape {c.shape}", flush=True)
        got = run_op(torch.from_numpy(c), device)
        np.testing.assert_array_equal(got, want, err_msg=f"{kind} {c.shape}")


@pytest.mark.parametrize("kind", jv_inputs.KINDS_LARGE)
def test_large_k_vs_oracle(kind, device):
    """K > 64: the global-memory kernel (cost outside LDS), at every
    chunk-count instantiation, rectangular both ways."""
    for n, m, c in jv_inputs.large_batches(kind):
        want = jv.jv_dense_batch(c)
        print(f"large kind {kind} shape {c.shape}", flush=True)
        got = run_op(torch.from_numpy(c), device)
        np.testing.assert_array_equal(got, want, err_msg=f"{kind} {c.shape}")


@pytest.mark.parametrize("kind", jv_inputs.KINDS_PADDED)
def test_padded_row_runs_vs_oracle(kind, device):
    """N < M: the padded rows (all 0) of the row reduction run in bulk while
    no dual falls, and the augmentation's padded start rows take the tied
    block's list 64 at a time.  Random shapes from a few padded rows to
    runs of several hundred (more than one 64-entry window), dense with and
    without the prefill workspace, and compact."""
    lib = _native.lib()
    for n, m, c in jv_inputs.padded_batches(kind):
        print(f"padded runs {kind} shape {c.shape}", flush=True)
        want = jv.jv_dense_batch(c)
        got = run_op(torch.from_numpy(c), device)
        np.testing.assert_array_equal(got, want, err_msg=f"{kind} {c.shape}")
        small = lib.tm_jv_workspace_bytes(4, n, m)
        got = _c_abi_solve(lib, lib.tm_jv_dense_batch_f32, c, small, device)
        np.testing.assert_array_equal(got, want, err_msg=f"plain workspace {kind} {c.shape}")
        got = _c_abi_solve(lib, lib.tm_jv_compact_batch_f32, c,
                           lib.tm_jv_workspace_bytes_prefill(4, n, m), device)
        np.testing.assert_array_equal(got, jv.jv_compact_batch(c),
                                      err_msg=f"compact {kind} {c.shape}")


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_c3_shape_other_seeds_vs_oracle(seed, device):
    """The C3 configuration (64, 512, 768), squared distances with 20 % +inf,
    at seeds beside the golden batch's: 256 padded rows per problem, so the
    row reduction's padded runs and the padded start rows' list run at full
    size."""
    c = workloads.jv_rect_masked(seed=seed)
    print(f"C3 shape seed {seed}", flush=True)
    np.testing.assert_array_equal(run_op(c, device), jv.jv_dense_batch(c.numpy()))


@pytest.mark.parametrize("shape", [(2100, 16, 16), (2050, 64, 64), (4, 100, 130)])
def test_signed_zero_through_statistics_pass(shape, device):
    """-0.0 (and +0.0 beside it) on the paths that take the statistics pass
    (B > 2048 at K <= 64, and K > 64): the pass flags -0.0, which keeps the
    K <= 64 kernel's displacement chains off, and the mapping stays the
    reference's."""
    rng = np.random.default_rng(zlib.crc32(repr(shape).encode()))
    c = jv_inputs.random_batch(rng, "signed_zero", *shape)
    print(f"signed zero {shape}", flush=True)
    np.testing.assert_array_equal(run_op(torch.from_numpy(c), device), jv.jv_dense_batch(c))


@pytest.mark.parametrize("kind", jv_inputs.KINDS_XL)
def test_xl_k_vs_oracle(kind, device):
    """1024 < K <= 2048: the 32-chunk instantiation without the row cache
    (every row-reduction step scans its row), through the op and through
    the C ABI with the prefill-sized workspace (which K > 1024 leaves
    unused)."""
    assert _native.jv_max_k() >= 2048
    lib = _native.lib()
    for n, m, c in jv_inputs.xl_batches(kind):
        want = jv.jv_dense_batch(c)
        print(f"xl kind {kind} shape {c.shape}", flush=True)
        got = run_op(torch.from_numpy(c), device)
        np.testing.assert_array_equal(got, want, err_msg=f"{kind} {c.shape}")
        ws = lib.tm_jv_workspace_bytes_prefill(*c.shape)
        assert ws == lib.tm_jv_workspace_bytes(*c.shape)
        got = _c_abi_solve(lib, lib.tm_jv_dense_batch_f32, c, ws, device)
        np.testing.assert_array_equal(got, want, err_msg=f"C ABI {kind} {c.shape}")


def _c_abi_solve(lib, entry, c: np.ndarray, ws_bytes: int, device) -> np.ndarray:
    b, n, m = c.shape
    dc = torch.from_numpy(c).to(device)
    out = torch.full((b, n), -7, dtype=torch.int64, device=device)
    ws = torch.full((ws_bytes,), 0xA5, dtype=torch.uint8, device=device)  # stale contents
    status = torch.zeros(2, dtype=torch.int32, device=device)
    stream = torch.cuda.current_stream(device).cuda_stream
    rc = entry(dc.data_ptr(), b, n, m, out.data_ptr(), ws.data_ptr(), ctypes.c_size_t(ws_bytes),
               status.data_ptr(), stream)
    assert rc == _native.TM_OK
    assert lib.tm_jv_check_status(status.data_ptr(), stream) == _native.TM_OK
    return out.cpu().numpy()


@pytest.mark.parametrize("kind", jv_inputs.KINDS_PREFILL)
def test_large_k_prefill_and_plain_workspace(kind, device):
    """K > 64 with the prefill workspace (column minima and row caches from
    many-wave launches) and with the minimum workspace (both in the solve's
    one wave): the same mapping as the oracle, dense and compact, at every
    chunk count, rectangular both ways."""
    lib = _native.lib()
    for n, m, c in jv_inputs.prefill_batches(kind):
        print(f"prefill kind {kind} shape {(4, n, m)}", flush=True)
        small = lib.tm_jv_workspace_bytes(4, n, m)
        full = lib.tm_jv_workspace_bytes_prefill(4, n, m)
        assert full > small
        want = jv.jv_dense_batch(c)
        for ws_bytes in (small, full):
            got = _c_abi_solve(lib, lib.tm_jv_dense_batch_f32, c, ws_bytes, device)
            np.testing.assert_array_equal(got, want, err_msg=f"{kind} {(n, m)} ws {ws_bytes}")
        want_c = jv.jv_compact_batch(c)
        for ws_bytes in (small, full):
            got = _c_abi_solve(lib, lib.tm_jv_compact_batch_f32, c, ws_bytes, device)
            np.testing.assert_array_equal(got, want_c, err_msg=f"compact {kind} {(n, m)}")


def test_plain_workspace_after_xl_layout(device):
    """Without the prefill the solve's row caches start empty: a regression
    test for slots left unset, whose stale LDS words (here the 2048-column
    layout's -1 owners and queue entries, NaN patterns as costs) once read
    as cache hits.  The cache-less solves run first on as many workgroups
    as the plain solves after them, so the latter inherit their LDS."""
    lib = _native.lib()
    rng = np.random.default_rng(77)
    xl = rng.random((64, 1100, 1100), dtype=np.float32)
    plain = rng.random((64, 70, 90), dtype=np.float32)
    want = jv.jv_dense_batch(plain)
    ws_small = lib.tm_jv_workspace_bytes(*plain.shape)
    for rep in range(2):
        print(f"xl then plain, round {rep}", flush=True)
        _c_abi_solve(lib, lib.tm_jv_dense_batch_f32, xl, lib.tm_jv_workspace_bytes(*xl.shape),
                     device)
        got = _c_abi_solve(lib, lib.tm_jv_dense_batch_f32, plain, ws_small, device)
        np.testing.assert_array_equal(got, want, err_msg=f"round {rep}")


def test_large_k_error_contracts_both_workspaces(device):
    """K > 64 with NaN or -inf: the prefill launches see the flags and write
    nothing, the solve fills -1 and the status decodes to TM_ERR_NAN /
    TM_ERR_NEG_INF (ops.cpp:67-93), with either workspace; an all-+inf
    problem (sentinel cost everywhere) beside finite ones still matches the
    oracle."""
    lib = _native.lib()
    stream = torch.cuda.current_stream(device).cuda_stream
    rng = np.random.default_rng(17)
    for bad, code in ((np.nan, _native.TM_ERR_NAN), (-np.inf, _native.TM_ERR_NEG_INF)):
        c = rng.random((3, 100, 130), dtype=np.float32)
        c[1, 50, 77] = bad
        print(f"large-K error contract {bad} (3, 100, 130)", flush=True)
        for ws_bytes in (lib.tm_jv_workspace_bytes(3, 100, 130),
                         lib.tm_jv_workspace_bytes_prefill(3, 100, 130)):
            dc = torch.from_numpy(c).to(device)
            out = torch.full((3, 100), -7, dtype=torch.int64, device=device)
            ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=device)
            status = torch.zeros(2, dtype=torch.int32, device=device)
            rc = lib.tm_jv_dense_batch_f32(dc.data_ptr(), 3, 100, 130, out.data_ptr(),
                                           ws.data_ptr(), ctypes.c_size_t(ws_bytes),
                                           status.data_ptr(), stream)
            assert rc == _native.TM_OK
            assert lib.tm_jv_check_status(status.data_ptr(), stream) == code
            assert (out.cpu().numpy() == -1).all()
    c = rng.random((3, 90, 120), dtype=np.float32)
    c[2] = np.inf
    print("large-K all-+inf problem (3, 90, 120)", flush=True)
    want = jv.jv_dense_batch(c)
    for ws_bytes in (lib.tm_jv_workspace_bytes(3, 90, 120),
                     lib.tm_jv_workspace_bytes_prefill(3, 90, 120)):
        got = _c_abi_solve(lib, lib.tm_jv_dense_batch_f32, c, ws_bytes, device)
        np.testing.assert_array_equal(got, want)


def test_c2_full_size_mapping_and_total_cost(device):
    cost = workloads.jv_uniform(1024, 64, 64, seed=0)
    want = jv.jv_dense_batch(cost.numpy())
    got = run_op(cost, device)
    np.testing.assert_array_equal(got, want)
    tot_got = assignment_cost(cost, torch.from_numpy(got))
    tot_want = assignment_cost(cost, torch.from_numpy(want))
    assert torch.equal(tot_got, tot_want)


def test_more_seeds_c2_shape(device):
    for seed in (1, 2, 3):
        cost = workloads.jv_uniform(1024, 64, 64, seed=seed)
        np.testing.assert_array_equal(run_op(cost, device), jv.jv_dense_batch(cost.numpy()))


def test_known_answers(device):
    inf = float("inf")
    cost = torch.tensor([[[1.0, inf], [inf, 1.0]], [[2.0, inf], [inf, 3.0]]])
    assert run_op(cost, device).tolist() == [[0, 1], [0, 1]]


def test_all_inf_problem(device):
    c = np.full((3, 5, 5), np.inf, np.float32)
    c[1] = np.random.default_rng(0).random((5, 5), dtype=np.float32)
    np.testing.assert_array_equal(run_op(torch.from_numpy(c), device), jv.jv_dense_batch(c))
    c = np.full((2, 4, 6), np.inf, np.float32)  # no finite cell at all: sentinel 1
    np.testing.assert_array_equal(run_op(torch.from_numpy(c), device), jv.jv_dense_batch(c))


def test_nan_and_neg_inf_rejected(device):
    c = torch.tensor([[[1.0, 2.0], [3.0, 4.0]], [[1.0, float("nan")], [3.0, 4.0]]])
    with pytest.raises(RuntimeError, match="NaN"):
        run_op(c, device)
    c = torch.tensor([[[1.0, 2.0], [3.0, 4.0]], [[1.0, float("-inf")], [3.0, 4.0]]])
    with pytest.raises(RuntimeError, match="-inf"):
        run_op(c, device)
    # the op keeps working afterwards
    c = torch.rand(4, 8, 8)
    np.testing.assert_array_equal(run_op(c, device), jv.jv_dense_batch(c.numpy()))


def test_empty_shapes(device):
    for shape in [(0, 4, 4), (3, 0, 4), (3, 4, 0)]:
        out = torch.ops.assignment.jonker_dense_batch(torch.empty(shape, device=device))
        assert out.shape == shape[:2] and (out == -1).all()


def test_float64_is_solved_in_float32(device):
    c64 = torch.rand(32, 20, 20, dtype=torch.float64)
    want = jv.jv_dense_batch(c64.to(torch.float32).numpy())
    np.testing.assert_array_equal(run_op(c64, device), want)


def test_non_contiguous_rejected(device):
    c = torch.rand(4, 8, 8, device=device).transpose(1, 2)
    with pytest.raises(RuntimeError, match="contiguous"):
        torch.ops.assignment.jonker_dense_batch(c)


def test_k_limit_enforced(device):
    k = _native.jv_max_k() + 1
    with pytest.raises(RuntimeError, match="K"):
        torch.ops.assignment.jonker_dense_batch(torch.rand(1, k, k, device=device))


def test_c_abi_direct(device):
    """The same kernel through the C ABI with raw device pointers."""
    lib = _native.lib()
    cost = workloads.jv_uniform(256, 48, 64, seed=4)
    dc = cost.to(device)
    out = torch.empty(256, 48, dtype=torch.int64, device=device)
    ws_bytes = lib.tm_jv_workspace_bytes(256, 48, 64)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=device)
    status = torch.zeros(2, dtype=torch.int32, device=device)
    stream = torch.cuda.current_stream(device).cuda_stream
    rc = lib.tm_jv_dense_batch_f32(dc.data_ptr(), 256, 48, 64, out.data_ptr(), ws.data_ptr(),
                                   ws_bytes, status.data_ptr(), stream)
    assert rc == _native.TM_OK
    assert lib.tm_jv_check_status(status.data_ptr(), stream) == _native.TM_OK
    np.testing.assert_array_equal(out.cpu().numpy(), jv.jv_dense_batch(cost.numpy()))
    # too-small workspace is refused without launching
    rc = lib.tm_jv_dense_batch_f32(dc.data_ptr(), 256, 48, 64, out.data_ptr(), ws.data_ptr(),
                                   ctypes.c_size_t(8), status.data_ptr(), stream)
    assert rc == _native.TM_ERR_WORKSPACE


def test_solve_dispatch_and_unpack(device):
    cost = workloads.jv_uniform(16, 12, 20, seed=6)
    packed = torchmatch_amd.assignment.solve(cost.to(device))
    np.testing.assert_array_equal(packed.cpu().numpy(), jv.jv_dense_batch(cost.numpy()))
    matches, ur, uc, n_matched = torchmatch_amd.assignment.solve(cost.to(device), unpack=True)
    assert (n_matched.cpu() == 12).all()
    assert matches.shape == (16, 12, 2)
    one = torchmatch_amd.assignment.solve(cost[0].to(device))
    np.testing.assert_array_equal(one.cpu().numpy(), jv.jv_dense_batch(cost[:1].numpy())[0])
    assert torchmatch_amd.assignment.resolve_backend(cost.to(device)) == "jonker_dense_batch"


@pytest.mark.parametrize(("n", "m", "p_inf"), [(12, 20, 0.0), (20, 12, 0.0), (30, 30, 0.6)])
def test_solve_2d_unpack(n, m, p_inf, device):
    """2-D solve(unpack=True): the device unpack on a batch of one, trimmed of
    its -1 padding as the reference's 2-D unpack returns it
    (assignment/_solve.py:124-164): matches (k, 2), unmatched rows (n - k),
    unmatched columns (m - k)."""
    cost = workloads.jv_rect_masked(B=1, N=n, M=m, p_inf=p_inf, seed=n * m)
    matches, ur, uc, nm = jv.unpack_packed(jv.jv_dense_batch(cost.numpy()), m)
    k = int(nm[0])
    got = torchmatch_amd.assignment.solve(cost[0].to(device), unpack=True)
    assert len(got) == 3
    np.testing.assert_array_equal(got[0].cpu().numpy(), matches[0, :k])
    np.testing.assert_array_equal(got[1].cpu().numpy(), ur[0, : n - k])
    np.testing.assert_array_equal(got[2].cpu().numpy(), uc[0, : m - k])


@pytest.mark.parametrize(("b", "n", "m", "p_inf"), [
    (64, 64, 64, 0.0), (32, 40, 64, 0.5), (16, 64, 30, 0.3), (8, 500, 768, 0.2),
    (4, 1, 1, 0.0), (3, 1000, 900, 0.9),
])
def test_unpacked_op_matches_cpu_format(b, n, m, p_inf, device):
    """assignment::jonker_dense_batch_unpacked on device: all four tensors equal
    the reference CPU op's (ops.cpp:291-417, restated in oracle.jv.unpack_packed)
    for the oracle's mapping of the same costs."""
    cost = workloads.jv_rect_masked(B=b, N=n, M=m, p_inf=p_inf, seed=n + m)
    print(f"unpacked {(b, n, m, p_inf)}", flush=True)
    want = jv.unpack_packed(jv.jv_dense_batch(cost.numpy()), m)
    got = torch.ops.assignment.jonker_dense_batch_unpacked(cost.to(device))
    for g, w in zip(got, want):
        np.testing.assert_array_equal(g.cpu().numpy(), w)
    via_solve = torchmatch_amd.assignment.solve(cost.to(device), unpack=True)
    for g, w in zip(via_solve, want):
        np.testing.assert_array_equal(g.cpu().numpy(), w)


def test_unpack_c_abi_direct(device):
    lib = _native.lib()
    packed = torch.tensor([[2, -1, 0], [-1, -1, -1], [0, 1, 2]], dtype=torch.int64,
                          device=device)
    outs = [torch.empty(3, 3, 2, dtype=torch.int64, device=device),
            torch.empty(3, 3, dtype=torch.int64, device=device),
            torch.empty(3, 4, dtype=torch.int64, device=device),
            torch.empty(3, dtype=torch.int64, device=device)]
    rc = lib.tm_jv_unpack_i64(packed.data_ptr(), 3, 3, 4, *[t.data_ptr() for t in outs],
                              torch.cuda.current_stream().cuda_stream)
    assert rc == _native.TM_OK
    torch.cuda.synchronize()
    for g, w in zip(outs, jv.unpack_packed(packed.cpu().numpy(), 4)):
        np.testing.assert_array_equal(g.cpu().numpy(), w)
    assert lib.tm_jv_unpack_i64(packed.data_ptr(), 3, 3, 5000, *[t.data_ptr() for t in outs],
                                None) == _native.TM_ERR_UNSUPPORTED_SHAPE


_GUARD_SCRIPT = textwrap.dedent(
    """
    import sys
    sys.path.insert(0, {root!r})
    import torch
    import torchmatch_amd  # noqa: F401
    cost = torch.rand(4, 8, 8, device="cuda", dtype=torch.float32)
    static_cost = cost.clone()
    graph = torch.cuda.CUDAGraph()
    try:
        with torch.cuda.graph(graph):
            torch.ops.assignment.jonker_dense_batch(static_cost)
    except RuntimeError as exc:
        message = str(exc)
        ok = "CUDA graph capture" in message and "jonker_dense_batch" in message
        print("GUARD_RAISED_OK" if ok else "GUARD_RAISED_WRONG_MESSAGE: " + message)
        sys.exit(0)
    print("GUARD_DID_NOT_RAISE")
    sys.exit(1)
    """
)


def test_graph_capture_guard(device):
    """Same contract as the reference's test_cudagraph_guard.py:42-91 (subprocess)."""
    res = subprocess.run(
        [sys.executable, "-c", _GUARD_SCRIPT.format(root=str(ROOT))],
        capture_output=True, text=True, timeout=120,
    )
    combined = f"stdout={res.stdout!r} stderr={res.stderr[-2000:]!r}"
    assert "GUARD_RAISED_OK" in res.stdout, combined
