"""Load the in-tree native extension and make sure the op schemas exist.

``_C.so`` carries the device kernels of ``assignment::jonker_dense_batch``,
``jonker_compact_batch`` and their ``_unpacked`` forms (CUDA dispatch key --
ROCm tensors report device type ``"cuda"``) and the private
``torchmatch_amd::sinkhorn_prepare`` / ``sinkhorn_iterate`` ops.  The
schemas of the ``assignment`` ops are owned by whoever defines the
``assignment`` library: the reference CPU extension when it is loaded
(``assignment/cpu/ops.cpp:486-498``), otherwise this module, with the same
texts and the same fake kernels as ``assignment/_loader.py:160-189``.

There is no fallback: if the extension is missing, :func:`load` raises.
"""

from __future__ import annotations

from pathlib import Path

import torch

_PKG = Path(__file__).resolve().parent
OPS_SO = _PKG / "_C.so"
CABI_SO = _PKG / "lib" / "libtorchmatch_amd.so"

# schema texts of assignment/cpu/ops.cpp:486-498 for the batched JV ops
BATCH_ROW_SCHEMAS = {
    "jonker_dense_batch": "jonker_dense_batch(Tensor costs) -> Tensor",
    "jonker_compact_batch": "jonker_compact_batch(Tensor costs) -> Tensor",
}
BATCH_UNPACKED_SCHEMAS = {
    "jonker_dense_batch_unpacked":
        "jonker_dense_batch_unpacked(Tensor costs) -> (Tensor, Tensor, Tensor, Tensor)",
    "jonker_compact_batch_unpacked":
        "jonker_compact_batch_unpacked(Tensor costs) -> (Tensor, Tensor, Tensor, Tensor)",
}

_state: dict[str, object] = {"loaded": False, "libs": []}


class ExtensionMissingError(RuntimeError):
    """The gfx950 extension was not built (run ``python torchmatch_amd/_build.py``)."""


def _has_op(namespace: str, name: str) -> bool:
    try:
        getattr(getattr(torch.ops, namespace), name)
    except (AttributeError, RuntimeError):
        return False
    return True


def _row_fake(costs: torch.Tensor) -> torch.Tensor:
    # assignment/_loader.py:160-169
    torch._check(costs.dim() == 3, lambda: "costs must be 3D (B, N, M)")
    return costs.new_empty(costs.size(0), costs.size(1), dtype=torch.long)


def _unpacked_fake(costs: torch.Tensor):
    # same shapes as the reference fake, assignment/_loader.py:172-189
    torch._check(costs.dim() == 3, lambda: "costs must be 3D (B, N, M)")
    b, n, m = costs.shape
    return (costs.new_empty(b, n, 2, dtype=torch.long),
            costs.new_empty(b, n, dtype=torch.long),
            costs.new_empty(b, m, dtype=torch.long),
            costs.new_empty(b, dtype=torch.long))


def _ensure_assignment_schema() -> None:
    for schemas, fake in ((BATCH_ROW_SCHEMAS, _row_fake),
                          (BATCH_UNPACKED_SCHEMAS, _unpacked_fake)):
        for name, schema in schemas.items():
            if _has_op("assignment", name):
                continue
            lib = torch.library.Library("assignment", "FRAGMENT")  # noqa: TOR901
            lib.define(schema)
            _state["libs"].append(lib)  # keep the registration alive
            torch.library.register_fake(f"assignment::{name}", fake, lib=lib)


def load() -> None:
    """Load ``_C.so`` once; raise :class:`ExtensionMissingError` if absent."""
    if _state["loaded"]:
        return
    if not OPS_SO.exists() or not CABI_SO.exists():
        msg = (
            f"torchmatch_amd native extension not found ({OPS_SO}, {CABI_SO}); "
            "build it with `python torchmatch_amd/_build.py` -- there is no "
            "non-native fallback"
        )
        raise ExtensionMissingError(msg)
    _ensure_assignment_schema()
    torch.ops.load_library(str(OPS_SO))
    _state["loaded"] = True


def native_library_paths() -> list[str]:
    """Paths of the native libraries this package loads (for diagnostics)."""
    return [str(OPS_SO), str(CABI_SO)]
