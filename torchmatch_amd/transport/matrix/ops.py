"""Direct handles for the ``torch.ops.transport.*`` ops this package provides
(reference: ``transport/matrix/ops.py:8-10``)."""

from __future__ import annotations

import torch

import torchmatch_amd.transport.matrix._sinkhorn  # noqa: F401  (registers the ops)

log_sinkhorn = torch.ops.transport.log_sinkhorn
sinkhorn_divergence = torch.ops.transport.sinkhorn_divergence
unbalanced_sinkhorn = torch.ops.transport.unbalanced_sinkhorn

__all__ = ["log_sinkhorn", "sinkhorn_divergence", "unbalanced_sinkhorn"]
