"""Random JV batches shared by the GPU parity tests and the CPU pins of the
oracle, so the oracle is checked against the reference build on exactly the
inputs the kernels are later compared with it on.

Each ``*_batches(kind)`` generator draws its batches from one
``numpy.random.default_rng`` seeded by the kind, in a fixed order, and yields
``(n, m, costs)``.
"""

from __future__ import annotations

import zlib

import numpy as np

KINDS_SMALL = ["uniform", "tied", "masked", "tied_masked", "negative", "huge"]
KINDS_LARGE = ["uniform", "tied", "masked", "tied_masked", "negative"]
KINDS_PREFILL = ["uniform", "tied", "masked", "tied_masked", "negative_masked"]
KINDS_COMPACT = ["uniform", "tied", "masked", "tied_masked", "negative", "huge", "big",
                 "signed_zero"]
KINDS_COMPACT_LARGE = ["uniform", "tied", "masked", "tied_masked", "negative", "huge", "big"]

# K <= 64 (the LDS-resident kernel), square and rectangular both ways
SMALL_SHAPES = [(64, 64), (1, 1), (1, 5), (5, 1), (2, 2), (17, 17), (31, 64), (64, 31),
                (63, 63), (40, 7), (7, 40), (33, 48)]
# K > 64: every chunk-count instantiation of the large-K kernel (2, 4, 8, 12
# and 16 chunks of 64 columns), rectangular both ways
LARGE_SHAPES = [(65, 65), (100, 80), (80, 100), (128, 128), (200, 130), (300, 300),
                (700, 768), (768, 600), (1000, 1024)]
PREFILL_SHAPES = [(65, 70), (130, 100), (100, 250), (300, 512), (512, 768), (768, 700),
                  (1024, 900)]
# K in (1024, 2048]: the 32-chunk instantiation without the row cache
KINDS_XL = ["uniform", "tied", "masked", "tied_masked"]
XL_SHAPES = [(1025, 1025), (1100, 1300), (2048, 1500), (1800, 2048)]


def random_batch(rng, kind: str, b: int, n: int, m: int) -> np.ndarray:
    if kind == "uniform":
        c = rng.random((b, n, m), dtype=np.float32)
    elif kind == "tied":
        c = rng.integers(0, 3, (b, n, m)).astype(np.float32)
    elif kind == "masked":
        c = rng.random((b, n, m), dtype=np.float32)
        c[rng.random((b, n, m)) < 0.5] = np.inf
    elif kind == "tied_masked":
        c = rng.integers(0, 2, (b, n, m)).astype(np.float32)
        c[rng.random((b, n, m)) < 0.3] = np.inf
    elif kind == "negative":
        c = (rng.random((b, n, m), dtype=np.float32) - 0.7) * 100.0
    elif kind == "negative_masked":
        # every finite cost <= -2, so the sentinel (max + 1) * (K + 1) lies
        # below all of them and +inf cells become column minima
        c = -(rng.random((b, n, m), dtype=np.float32) * 100.0 + 2.0)
        c[rng.random((b, n, m)) < 0.3] = np.inf
    elif kind == "huge":  # beyond 1e15: lane-serial path
        c = rng.random((b, n, m), dtype=np.float32) * np.float32(3e16)
    elif kind == "big":  # 1e12 .. 1e15: serial for compact, wave path for dense
        c = rng.random((b, n, m), dtype=np.float32) * np.float32(5e13)
        c[rng.random((b, n, m)) < 0.1] = np.inf
    elif kind == "signed_zero":
        c = rng.integers(-1, 2, (b, n, m)).astype(np.float32) * np.float32(0.0)
        c[rng.random((b, n, m)) < 0.5] = np.float32(1.0)
    else:
        raise ValueError(kind)
    return c


def small_batches(kind: str):
    rng = np.random.default_rng(zlib.crc32(kind.encode()))
    for n, m in SMALL_SHAPES:
        yield n, m, random_batch(rng, kind, 64 if kind != "huge" else 8, n, m)


def large_batches(kind: str):
    rng = np.random.default_rng(zlib.crc32(("large" + kind).encode()))
    for n, m in LARGE_SHAPES:
        yield n, m, random_batch(rng, kind, 6, n, m)


def prefill_batches(kind: str):
    rng = np.random.default_rng(zlib.crc32(("prefill" + kind).encode()))
    for n, m in PREFILL_SHAPES:
        yield n, m, random_batch(rng, kind, 4, n, m)


# N < M with padded-row runs from a few rows to several hundred
KINDS_PADDED = ["uniform", "tied", "masked", "tied_masked", "negative_masked"]


def padded_batches(kind: str):
    rng = np.random.default_rng(zlib.crc32(("padded" + kind).encode()))
    shapes = [(65, 1000), (70, 200), (129, 130), (200, 460)]
    shapes += [(int(n), int(rng.integers(n + 1, min(1024, 3 * n) + 1)))
               for n in rng.integers(40, 300, 6)]
    for n, m in shapes:
        yield n, m, random_batch(rng, kind, 4, n, m)


def xl_batches(kind: str):
    rng = np.random.default_rng(zlib.crc32(("xl" + kind).encode()))
    for n, m in XL_SHAPES:
        yield n, m, random_batch(rng, kind, 2, n, m)


def compact_small_batches(kind: str, kmax: int = 64):
    rng = np.random.default_rng(zlib.crc32(b"compact-gpu-" + kind.encode()))
    shapes = [(64, kmax, kmax), (64, 40, kmax), (64, kmax, 23), (128, 17, 17), (128, 5, 5),
              (64, 1, 1), (64, 2, 2), (64, 3, 7)]
    for b, n, m in shapes:
        yield n, m, random_batch(rng, kind, b, n, m)


def compact_large_batches(kind: str):
    rng = np.random.default_rng(zlib.crc32(b"compact-large-" + kind.encode()))
    shapes = [(16, 65, 65), (8, 100, 130), (8, 130, 100), (6, 300, 300), (3, 700, 768)]
    if kind not in ("huge", "big"):
        shapes.append((2, 1024, 1000))
    for b, n, m in shapes:
        yield n, m, random_batch(rng, kind, b, n, m)
