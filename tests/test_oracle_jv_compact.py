"""Pins the compact JV oracle (jvoc_square in oracle/jv_oracle.c, the
restatement of jonker_compact_core.h:20-252 behind ops.cpp:431-433) before the
GPU kernel is compared to it.

* against the reference's compact solver compiled from its own header
  (oracle/_ref/libjv_ref.so) on random, tied, masked and negative batches,
  square and rectangular;
* against the committed golden fixtures ("compact" mappings written from
  that build by tests/golden/make_jv_golden.py);
* against scipy.optimize.linear_sum_assignment (optimal total cost) and brute
  force over permutations (K <= 7);
* the tie rules have teeth: on tied batches the compact mappings differ from
  the dense solver's, so a restatement that fell back to the dense rules
  would fail the golden and reference checks.
"""

from __future__ import annotations

import itertools
import json
import zlib
from pathlib import Path

import numpy as np
import pytest

from oracle import jv
import jv_inputs
import workloads

GOLDEN = Path(__file__).resolve().parent / "golden"


def _cost_total(c: np.ndarray, mapping: np.ndarray) -> np.ndarray:
    valid = mapping >= 0
    picked = np.take_along_axis(c, np.clip(mapping, 0, None)[..., None], axis=2)[..., 0]
    return np.where(valid, picked, 0.0).astype(np.float64).sum(axis=1)


def _batch(kind: str, rng, b, n, m):
    if kind == "uniform":
        return rng.random((b, n, m), dtype=np.float32)
    if kind == "tied":
        return rng.integers(0, 3, (b, n, m)).astype(np.float32)
    if kind == "masked":
        c = rng.random((b, n, m), dtype=np.float32)
        c[rng.random((b, n, m)) < 0.6] = np.inf
        return c
    if kind == "tied_masked":
        c = rng.integers(0, 2, (b, n, m)).astype(np.float32)
        c[rng.random((b, n, m)) < 0.3] = np.inf
        return c
    if kind == "negative":
        return (rng.standard_normal((b, n, m)) * 50).astype(np.float32)
    raise ValueError(kind)


def test_known_answers():
    inf = np.inf
    c = np.array([[[1.0, inf], [inf, 1.0]], [[2.0, inf], [inf, 3.0]]], dtype=np.float32)
    assert jv.jv_compact_batch(c).tolist() == [[0, 1], [0, 1]]
    with pytest.raises(jv.OracleError, match="NaN"):
        jv.jv_compact_batch(np.array([[[1.0, np.nan], [3.0, 4.0]]], np.float32))
    with pytest.raises(jv.OracleError, match="-inf"):
        jv.jv_compact_batch(np.array([[[1.0, -inf], [3.0, 4.0]]], np.float32))
    assert (jv.jv_compact_batch(np.zeros((2, 3, 0), np.float32)) == -1).all()


@pytest.mark.skipif(not jv.ref_available(), reason="reference build (oracle/_ref) absent")
@pytest.mark.parametrize("kind", ["uniform", "tied", "masked", "tied_masked", "negative"])
def test_oracle_matches_reference_build(kind):
    rng = np.random.default_rng(zlib.crc32(b"compact-" + kind.encode()))
    for _ in range(25):
        b, n, m = 32, int(rng.integers(1, 70)), int(rng.integers(1, 70))
        c = _batch(kind, rng, b, n, m)
        np.testing.assert_array_equal(jv.jv_compact_batch(c), jv.ref_jv_compact_batch(c))
    c = _batch(kind, rng, 4, 300, 300)
    np.testing.assert_array_equal(jv.jv_compact_batch(c), jv.ref_jv_compact_batch(c))


@pytest.mark.skipif(not jv.ref_available(), reason="reference build (oracle/_ref) absent")
@pytest.mark.parametrize("kind", jv_inputs.KINDS_COMPACT)
def test_oracle_matches_reference_build_on_gpu_inputs(kind):
    """The exact batches the compact GPU tests compare the kernels with this
    oracle on (tests/test_jv_compact_gpu.py), K <= 64 and 64 < K <= 1024:
    oracle == reference build."""
    for n, m, c in jv_inputs.compact_small_batches(kind):
        np.testing.assert_array_equal(jv.jv_compact_batch(c), jv.ref_jv_compact_batch(c),
                                      err_msg=f"{kind} {c.shape}")
    if kind in jv_inputs.KINDS_COMPACT_LARGE:
        for n, m, c in jv_inputs.compact_large_batches(kind):
            np.testing.assert_array_equal(jv.jv_compact_batch(c), jv.ref_jv_compact_batch(c),
                                          err_msg=f"large {kind} {c.shape}")


def _golden_cases():
    index = json.loads((GOLDEN / "jv_golden.json").read_text())
    return sorted(index.items())


@pytest.mark.parametrize(("name", "meta"), _golden_cases(), ids=[n for n, _ in _golden_cases()])
def test_oracle_matches_golden(name, meta):
    cost = getattr(workloads, meta["generator"])(**meta["kwargs"])
    assert workloads.sha256(cost) == meta["sha256"], "input generator drifted"
    want = np.load(GOLDEN / meta["file"])["compact"].astype(np.int64)
    np.testing.assert_array_equal(jv.jv_compact_batch(cost.numpy()), want)


def test_optimal_cost_against_scipy():
    sp = pytest.importorskip("scipy.optimize")
    rng = np.random.default_rng(17)
    for n, m in [(16, 16), (20, 33), (33, 20), (64, 64)]:
        c = rng.random((16, n, m), dtype=np.float32)
        got = _cost_total(c, jv.jv_compact_batch(c))
        for b in range(c.shape[0]):
            r, k = sp.linear_sum_assignment(c[b].astype(np.float64))
            assert got[b] == pytest.approx(float(c[b][r, k].astype(np.float64).sum()), abs=1e-4)


def test_optimal_cost_brute_force():
    rng = np.random.default_rng(21)
    for k in range(1, 8):
        c = rng.integers(0, 5, (20, k, k)).astype(np.float32)
        got = _cost_total(c, jv.jv_compact_batch(c))
        for b in range(c.shape[0]):
            best = min(
                sum(float(c[b, i, p[i]]) for i in range(k))
                for p in itertools.permutations(range(k))
            )
            assert got[b] == best


def test_tie_rules_differ_from_dense():
    c = workloads.integer_tied(64, 32, 32, seed=8, hi=3).numpy()
    compact, dense = jv.jv_compact_batch(c), jv.jv_dense_batch(c)
    assert (compact != dense).any(axis=1).sum() > 32
    np.testing.assert_array_equal(_cost_total(c, compact), _cost_total(c, dense))
