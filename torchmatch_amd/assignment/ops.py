"""Direct access to the ``torch.ops.assignment.*`` op this package provides.

Mirrors ``assignment/ops.py:17-28`` of the reference for the one op on the
gfx950 path; the reference's other CPU / CUDA solvers are not part of it.
"""

from __future__ import annotations

import torch

from torchmatch_amd._loader import load as _load

_load()

jonker_dense_batch = torch.ops.assignment.jonker_dense_batch

__all__ = ["jonker_dense_batch"]
