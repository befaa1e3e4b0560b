"""Write the JV golden fixtures from the reference's own compiled solvers.

Runs in the build container only (needs oracle/_ref/libjv_ref.so, which
oracle/Makefile compiles from the reference's jonker_dense_core.cpp and
jonker_compact_core.h):

    make -C oracle && python tests/golden/make_jv_golden.py

Each fixture stores the workload recipe (generator + seed + shape), the
sha256 of the float32 input bytes, and the reference int64 row->col mappings
of jonker_dense_batch ("mapping") and jonker_compact_batch ("compact") in the
narrowest integer type that holds them.  Tests regenerate the input
from the recipe, check the sha256, and compare mappings.
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import jv  # noqa: E402
import workloads  # noqa: E402

OUT = Path(__file__).resolve().parent

# name -> (generator, kwargs)
CASES: dict[str, tuple[str, dict]] = {
    "c1_uniform_8x16x16": ("jv_uniform", {"B": 8, "N": 16, "M": 16, "seed": 0}),
    "c2_uniform_1024x64x64": ("jv_uniform", {"B": 1024, "N": 64, "M": 64, "seed": 0}),
    "c3_rect_masked_64x512x768": ("jv_rect_masked", {"seed": 0}),
    "tied_256x64x64": ("integer_tied", {"B": 256, "N": 64, "M": 64, "seed": 1}),
    "tied_rect_256x40x64": ("integer_tied", {"B": 256, "N": 40, "M": 64, "seed": 2, "hi": 4}),
    "tied_rect_256x64x23": ("integer_tied", {"B": 256, "N": 64, "M": 23, "seed": 3, "hi": 3}),
    "gated_sparse_256x64": ("gated_sparse", {"B": 256, "n": 64, "seed": 4}),
    "gated_sparse_512x17": ("gated_sparse", {"B": 512, "n": 17, "seed": 5}),
}


def make_input(name: str):
    gen, kw = CASES[name]
    return getattr(workloads, gen)(**kw)


def main() -> None:
    if not jv.ref_available():
        raise SystemExit("oracle/_ref/libjv_ref.so missing: run `make -C oracle` first")
    index = {}
    for name, (gen, kw) in CASES.items():
        cost = make_input(name)
        ref = jv.ref_jv_dense_batch(cost.numpy())
        compact = jv.ref_jv_compact_batch(cost.numpy())
        m = cost.shape[2]
        dtype = np.int8 if m <= 127 else np.int16
        np.savez_compressed(OUT / f"jv_{name}.npz", mapping=ref.astype(dtype),
                            compact=compact.astype(dtype))
        index[name] = {
            "generator": gen,
            "kwargs": kw,
            "shape": list(cost.shape),
            "sha256": workloads.sha256(cost),
            "file": f"jv_{name}.npz",
            "unmatched": int((ref < 0).sum()),
            "compact_unmatched": int((compact < 0).sum()),
            "compact_differs": int((compact != ref).any(axis=1).sum()),
        }
        print(name, cost.shape, "unmatched:", int((ref < 0).sum()),
              "compact differs on", int((compact != ref).any(axis=1).sum()), "problems")
    (OUT / "jv_golden.json").write_text(json.dumps(index, indent=2) + "\n")


if __name__ == "__main__":
    main()
