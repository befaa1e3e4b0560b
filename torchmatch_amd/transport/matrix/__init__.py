"""Cost-matrix Sinkhorn on MI355X (mirrors ``torchmatch.transport.matrix``).

Registers ``torch.ops.transport.log_sinkhorn`` and
``torch.ops.transport.unbalanced_sinkhorn`` with the reference's schemas and a
gfx950 kernel for device tensors, and provides the ``solve`` dispatcher.
"""

from __future__ import annotations

from torchmatch_amd._loader import load as _load

_load()

from torchmatch_amd.transport.matrix import ops  # noqa: E402
from torchmatch_amd.transport.matrix._solve import (  # noqa: E402
    Backend,
    marginal_error,
    solve,
)

__all__ = ["Backend", "marginal_error", "ops", "solve"]
