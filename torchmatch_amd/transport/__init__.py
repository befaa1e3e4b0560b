"""Optimal-transport solvers on MI355X (mirrors ``torchmatch.transport``).

Only the cost-matrix face (:mod:`torchmatch_amd.transport.matrix`) is part of
this package; the reference's Triton point-cloud face is not.
"""

from __future__ import annotations

from torchmatch_amd.transport import matrix

__all__ = ["matrix"]
