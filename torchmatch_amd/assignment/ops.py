"""Direct access to the ``torch.ops.assignment.*`` ops this package provides.

Mirrors ``assignment/ops.py:17-28`` of the reference for the batched JV ops
on the gfx950 path (device kernels of the same op names); the reference's
single-problem and other CPU / CUDA solvers are not part of it.
"""

from __future__ import annotations

import torch

from torchmatch_amd._loader import load as _load

_load()

_OPS = torch.ops.assignment

jonker_dense_batch = _OPS.jonker_dense_batch
jonker_compact_batch = _OPS.jonker_compact_batch
jonker_dense_batch_unpacked = _OPS.jonker_dense_batch_unpacked
jonker_compact_batch_unpacked = _OPS.jonker_compact_batch_unpacked

__all__ = [
    "jonker_compact_batch",
    "jonker_compact_batch_unpacked",
    "jonker_dense_batch",
    "jonker_dense_batch_unpacked",
]
