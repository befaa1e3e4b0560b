"""Batched linear assignment on MI355X (mirrors ``torchmatch.assignment``).

Public surface (same names as the reference, ``assignment/__init__.py:152-159``):

- :func:`solve` -- dispatcher; device tensors go to the gfx950 JV kernel;
- :class:`Backend` -- backend choices accepted by :func:`solve`;
- :func:`resolve_backend` -- the op :func:`solve` would call;
- :func:`assignment_cost` -- total cost of a row->col mapping;
- :mod:`ops` -- ``torch.ops.assignment.*`` handles provided here.
"""

from __future__ import annotations

from torchmatch_amd._loader import load as _load

_load()

from torchmatch_amd.assignment import ops  # noqa: E402
from torchmatch_amd.assignment._cost import assignment_cost  # noqa: E402
from torchmatch_amd.assignment._solve import Backend, resolve_backend, solve  # noqa: E402

__all__ = ["Backend", "assignment_cost", "ops", "resolve_backend", "solve"]
