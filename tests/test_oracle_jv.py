"""Pins the JV oracle (oracle/jv_oracle.c) before anything is compared to it.

* against the reference's own solver compiled from its source
  (oracle/_ref/libjv_ref.so, built by oracle/Makefile) on random, tied and
  masked batches, square and rectangular;
* against the committed golden fixtures (written from that same reference
  build by tests/golden/make_jv_golden.py);
* against scipy.optimize.linear_sum_assignment (optimal total cost) and
  brute force over permutations (K <= 7), which pin optimality independently
  of the reference;
* against the reference tests' known answers (test_lap_inf_mask.py:50-126)
  and the sentinel rule (ops.cpp:67-93).
"""

from __future__ import annotations

import itertools
import zlib
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import jv
import jv_inputs
import workloads

GOLDEN = Path(__file__).resolve().parent / "golden"


def _cost_total(c: np.ndarray, mapping: np.ndarray) -> np.ndarray:
    b, n, _ = c.shape
    valid = mapping >= 0
    picked = np.take_along_axis(c, np.clip(mapping, 0, None)[..., None], axis=2)[..., 0]
    return np.where(valid, picked, 0.0).astype(np.float64).sum(axis=1)


def test_known_answers_from_reference_tests():
    inf = np.inf
    c = np.array([[[1.0, inf], [inf, 1.0]], [[2.0, inf], [inf, 3.0]]], dtype=np.float32)
    assert jv.jv_dense_batch(c).tolist() == [[0, 1], [0, 1]]
    with pytest.raises(jv.OracleError, match="NaN"):
        jv.jv_dense_batch(np.array([[[1.0, 2.0], [3.0, 4.0]], [[1.0, np.nan], [3.0, 4.0]]]))
    with pytest.raises(jv.OracleError, match="-inf"):
        jv.jv_dense_batch(np.array([[[1.0, 2.0], [3.0, 4.0]], [[1.0, -inf], [3.0, 4.0]]]))


def test_empty_shapes_give_minus_one():
    assert jv.jv_dense_batch(np.zeros((0, 3, 3), np.float32)).shape == (0, 3)
    out = jv.jv_dense_batch(np.zeros((2, 3, 0), np.float32))
    assert out.shape == (2, 3) and (out == -1).all()


def test_sentinel_rule():
    c = np.array([[[1.5, np.inf], [np.inf, -2.0]]], dtype=np.float32)
    assert jv.sentinel(c) == np.float32((np.float32(1.5) + np.float32(1)) * np.float32(3))
    assert jv.sentinel(np.full((1, 2, 3), np.inf, np.float32)) == 1.0


@pytest.mark.skipif(not jv.ref_available(), reason="reference build (oracle/_ref) absent")
@pytest.mark.parametrize("kind", ["uniform", "tied", "masked", "tied_masked"])
def test_oracle_matches_reference_build(kind):
    rng = np.random.default_rng(zlib.crc32(kind.encode()))
    for _ in range(25):
        b, n, m = 32, int(rng.integers(1, 48)), int(rng.integers(1, 48))
        if kind == "uniform":
            c = rng.random((b, n, m), dtype=np.float32)
        elif kind == "tied":
            c = rng.integers(0, 3, (b, n, m)).astype(np.float32)
        elif kind == "masked":
            c = rng.random((b, n, m), dtype=np.float32)
            c[rng.random((b, n, m)) < 0.6] = np.inf
        else:
            c = rng.integers(0, 2, (b, n, m)).astype(np.float32)
            c[rng.random((b, n, m)) < 0.3] = np.inf
        np.testing.assert_array_equal(jv.jv_dense_batch(c), jv.ref_jv_dense_batch(c))


@pytest.mark.skipif(not jv.ref_available(), reason="reference build (oracle/_ref) absent")
@pytest.mark.parametrize("kind", jv_inputs.KINDS_SMALL)
def test_oracle_matches_reference_build_on_small_k_gpu_inputs(kind):
    """The exact K <= 64 batches the GPU tests compare the kernel with the
    oracle on (tests/test_jv_gpu.py): oracle == reference build."""
    for n, m, c in jv_inputs.small_batches(kind):
        np.testing.assert_array_equal(jv.jv_dense_batch(c), jv.ref_jv_dense_batch(c),
                                      err_msg=f"{kind} {c.shape}")


@pytest.mark.skipif(not jv.ref_available(), reason="reference build (oracle/_ref) absent")
@pytest.mark.parametrize("kind", jv_inputs.KINDS_LARGE)
def test_oracle_matches_reference_build_on_large_k_gpu_inputs(kind):
    """K = 65 ... 1024, rectangular both ways, negative costs: the exact
    batches of the GPU large-K tests, oracle == reference build."""
    for n, m, c in jv_inputs.large_batches(kind):
        np.testing.assert_array_equal(jv.jv_dense_batch(c), jv.ref_jv_dense_batch(c),
                                      err_msg=f"{kind} {c.shape}")


@pytest.mark.skipif(not jv.ref_available(), reason="reference build (oracle/_ref) absent")
@pytest.mark.parametrize("kind", jv_inputs.KINDS_PREFILL)
def test_oracle_matches_reference_build_on_prefill_gpu_inputs(kind):
    """The batches of the GPU prefill / plain-workspace test, dense and
    compact solvers."""
    for n, m, c in jv_inputs.prefill_batches(kind):
        np.testing.assert_array_equal(jv.jv_dense_batch(c), jv.ref_jv_dense_batch(c),
                                      err_msg=f"dense {kind} {c.shape}")
        np.testing.assert_array_equal(jv.jv_compact_batch(c), jv.ref_jv_compact_batch(c),
                                      err_msg=f"compact {kind} {c.shape}")


@pytest.mark.skipif(not jv.ref_available(), reason="reference build (oracle/_ref) absent")
@pytest.mark.parametrize("seed", [1, 2, 3])
def test_oracle_matches_reference_build_on_c3_seeds(seed):
    """The C3-shape batches of the GPU test beside the golden one."""
    c = workloads.jv_rect_masked(seed=seed).numpy()
    np.testing.assert_array_equal(jv.jv_dense_batch(c), jv.ref_jv_dense_batch(c))


@pytest.mark.skipif(not jv.ref_available(), reason="reference build (oracle/_ref) absent")
@pytest.mark.parametrize("kind", jv_inputs.KINDS_PADDED)
def test_oracle_matches_reference_build_on_padded_gpu_inputs(kind):
    """The batches of the GPU padded-row-run test, dense and compact."""
    for n, m, c in jv_inputs.padded_batches(kind):
        np.testing.assert_array_equal(jv.jv_dense_batch(c), jv.ref_jv_dense_batch(c),
                                      err_msg=f"dense {kind} {c.shape}")
        np.testing.assert_array_equal(jv.jv_compact_batch(c), jv.ref_jv_compact_batch(c),
                                      err_msg=f"compact {kind} {c.shape}")


@pytest.mark.skipif(not jv.ref_available(), reason="reference build (oracle/_ref) absent")
@pytest.mark.parametrize("kind", jv_inputs.KINDS_XL)
def test_oracle_matches_reference_build_on_xl_gpu_inputs(kind):
    """K = 1025 ... 2048 (the cache-less instantiation), rectangular both
    ways: the batches of the GPU K > 1024 tests, dense and compact."""
    for n, m, c in jv_inputs.xl_batches(kind):
        np.testing.assert_array_equal(jv.jv_dense_batch(c), jv.ref_jv_dense_batch(c),
                                      err_msg=f"dense {kind} {c.shape}")
        np.testing.assert_array_equal(jv.jv_compact_batch(c), jv.ref_jv_compact_batch(c),
                                      err_msg=f"compact {kind} {c.shape}")


def _golden_cases():
    index = json.loads((GOLDEN / "jv_golden.json").read_text())
    return sorted(index.items())


@pytest.mark.parametrize(("name", "meta"), _golden_cases(), ids=[n for n, _ in _golden_cases()])
def test_oracle_matches_golden(name, meta):
    cost = getattr(workloads, meta["generator"])(**meta["kwargs"])
    assert workloads.sha256(cost) == meta["sha256"], "input generator drifted"
    want = np.load(GOLDEN / meta["file"])["mapping"].astype(np.int64)
    np.testing.assert_array_equal(jv.jv_dense_batch(cost.numpy()), want)


def test_optimal_cost_against_scipy():
    sp = pytest.importorskip("scipy.optimize")
    rng = np.random.default_rng(7)
    for n, m in [(16, 16), (20, 33), (33, 20), (64, 64)]:
        c = rng.random((16, n, m), dtype=np.float32)
        got = _cost_total(c, jv.jv_dense_batch(c))
        for b in range(c.shape[0]):
            r, k = sp.linear_sum_assignment(c[b].astype(np.float64))
            assert got[b] == pytest.approx(float(c[b][r, k].astype(np.float64).sum()), abs=1e-4)


def test_optimal_cost_brute_force():
    rng = np.random.default_rng(11)
    for k in range(1, 8):
        c = rng.integers(0, 5, (20, k, k)).astype(np.float32)
        got = _cost_total(c, jv.jv_dense_batch(c))
        for b in range(c.shape[0]):
            best = min(
                sum(float(c[b, i, p[i]]) for i in range(k))
                for p in itertools.permutations(range(k))
            )
            assert got[b] == best


def test_mapping_is_partial_permutation():
    c = workloads.jv_uniform(64, 20, 30, seed=3).numpy()
    out = jv.jv_dense_batch(c)
    for row in out:
        assert len(set(row.tolist())) == len(row)
        assert ((row >= 0) & (row < 30)).all()
    c = workloads.jv_uniform(64, 30, 20, seed=3).numpy()
    out = jv.jv_dense_batch(c)
    assert ((out >= 0).sum(axis=1) == 20).all()


def test_planted_mistake_is_caught():
    """A transposed operand must not pass the brute-force check (sanity of the pin)."""
    rng = np.random.default_rng(5)
    c = rng.random((50, 5, 5), dtype=np.float32)
    wrong = jv.jv_dense_batch(np.ascontiguousarray(c.transpose(0, 2, 1)))
    right = jv.jv_dense_batch(c)
    assert not np.array_equal(_cost_total(c, wrong), _cost_total(c, right))


def test_counted_run_matches_plain_run():
    c = workloads.jv_uniform(16, 64, 64, seed=9).numpy()
    out, counts = jv.jv_dense_batch_counted(c)
    np.testing.assert_array_equal(out, jv.jv_dense_batch(c))
    assert (counts[:, 0] >= 64 * 64).all()


def test_bench_relaxation_count():
    """bench.py prices the JV LDS roofline in relaxations on C2 seed 0; the
    constant it carries must be what the counted oracle run gives."""
    import bench

    c = workloads.jv_uniform(1024, 64, 64, seed=0).numpy()
    out, counts = jv.jv_dense_batch_counted(c)
    assert int(counts[:, 0].sum()) == bench.JV_C2_RELAXATIONS
    # every problem scans its full K x K tile at least once (column reduction)
    assert (counts[:, 0] >= 64 * 64).all()


def test_bench_critical_steps():
    """bench.py floors the JV launch at the slowest C2 seed-0 problem's
    sequential search steps under the kernel's certified path; the work model
    gives the same mappings as the reference on that batch (its optimum is
    unique everywhere) and the constant bench.py carries."""
    import bench

    c = workloads.jv_uniform(1024, 64, 64, seed=0).numpy()
    out, counts = jv.sap_batch_counted(c)
    np.testing.assert_array_equal(out, jv.jv_dense_batch(c))
    steps = counts[:, 1] + counts[:, 2]
    assert int(steps.max()) == bench.JV_C2_CRITICAL_STEPS
    # the reference order's augmenting row reduction is skipped: fewer
    # relaxations than the reference's count
    assert int(counts[:, 0].sum()) < bench.JV_C2_RELAXATIONS


def test_bench_c3_critical_steps():
    """bench.py floors the C3 batch at its slowest problem's sequential steps
    in the reference's order (augmenting row reduction steps + paths + rows
    scanned in the paths), which the K = 768 kernel replays one after another.
    The step counter is checked on hand cases first."""
    import bench

    # column reduction settles a strictly diagonal problem: no further step
    eye = (1.0 - np.eye(5, dtype=np.float32))[None]
    _, st = jv.jv_dense_batch_steps(eye)
    assert st.tolist() == [[0, 0, 0]]
    # by hand: columns 1 and 2 take their minimum rows 0 and 1 (column 1
    # outranks column 0 for row 0); row 2 stays free and one row-reduction
    # step gives it column 0 (reduced costs 0, 1, 2: no displacement)
    crowd = np.array([[[0, 5, 6], [0, 7, 5], [0, 6, 7]]], dtype=np.float32)
    out, st = jv.jv_dense_batch_steps(crowd)
    assert st.tolist() == [[1, 0, 0]]
    assert out.tolist() == [[1, 2, 0]]
    c = workloads.jv_rect_masked().numpy()
    out, st = jv.jv_dense_batch_steps(c)
    np.testing.assert_array_equal(out, jv.jv_dense_batch(c))
    assert int(st.sum(axis=1).max()) == bench.JV_C3_CRITICAL_STEPS


def test_unpack_restatement_known_cases():
    """Hand-worked unpacks (ops.cpp:387-414): row order of matches, increasing
    unmatched rows / columns, -1 padding."""
    packed = np.array([[2, -1, 0], [-1, -1, -1], [0, 1, 2]])
    matches, ur, uc, nm = jv.unpack_packed(packed, 4)
    np.testing.assert_array_equal(nm, [2, 0, 3])
    np.testing.assert_array_equal(matches[0], [[0, 2], [2, 0], [-1, -1]])
    np.testing.assert_array_equal(ur[0], [1, -1, -1])
    np.testing.assert_array_equal(uc[0], [1, 3, -1, -1])
    np.testing.assert_array_equal(matches[1], [[-1, -1]] * 3)
    np.testing.assert_array_equal(ur[1], [0, 1, 2])
    np.testing.assert_array_equal(uc[1], [0, 1, 2, 3])
    np.testing.assert_array_equal(matches[2], [[0, 0], [1, 1], [2, 2]])
    np.testing.assert_array_equal(uc[2], [3, -1, -1, -1])


def test_unpack_restatement_invariants():
    """On real solves: every row is matched or unmatched exactly once, every
    column used at most once, and n_matches counts the non-negative entries."""
    c = workloads.jv_rect_masked(B=4, N=30, M=45, p_inf=0.6, seed=3).numpy()
    packed = jv.jv_dense_batch(c)
    matches, ur, uc, nm = jv.unpack_packed(packed, c.shape[2])
    for k in range(c.shape[0]):
        rows = set(matches[k, : nm[k], 0]) | set(ur[k, : 30 - nm[k]])
        assert rows == set(range(30))
        cols = list(matches[k, : nm[k], 1]) + list(uc[k, : 45 - nm[k]])
        assert sorted(cols) == list(range(45))
        assert nm[k] == (packed[k] >= 0).sum()


def test_torch_input_roundtrip():
    c = torch.rand(4, 6, 6, generator=torch.Generator().manual_seed(0))
    assert jv.jv_dense_batch(c.numpy()).shape == (4, 6)
