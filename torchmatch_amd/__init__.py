"""torchmatch_amd -- MI355X (gfx950) kernels for torchmatch's data-parallel solvers.

Drop-in device kernels for two of torchmatch's ops, behind the same names
and schemas:

* ``torch.ops.assignment.jonker_dense_batch`` -- batched Jonker-Volgenant
  assignment, bit-identical to the reference CPU op;
* ``torch.ops.transport.log_sinkhorn`` / ``unbalanced_sinkhorn`` --
  log-domain Sinkhorn transport plans.

``torchmatch_amd.assignment.solve`` and ``torchmatch_amd.transport.matrix.solve``
mirror ``torchmatch.assignment.solve`` and ``torchmatch.transport.matrix.solve``.
The C ABI underneath is declared in ``include/torchmatch_amd.h``.
"""

from __future__ import annotations

from torchmatch_amd._loader import ExtensionMissingError, load

load()

from torchmatch_amd import assignment, transport  # noqa: E402

__all__ = ["ExtensionMissingError", "assignment", "load", "transport"]
