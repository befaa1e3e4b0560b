"""ctypes front-end to the JV parity checkers (TEST INFRASTRUCTURE ONLY).

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg
may import this module.  It loads:

* ``oracle/libjv_oracle.so`` -- the C restatement in ``jv_oracle.c`` of the
  reference's float32 ``jonker_dense_batch`` (ops.cpp:67-93,176-289,
  jonker_dense_core.cpp:15-60, jonker_dense_flat.h:27-274) and
  ``jonker_compact_batch`` (ops.cpp:431-433, jonker_compact_core.h:20-301);
* ``oracle/_ref/libjv_ref.so`` -- the reference's own ``jonker_dense_core.cpp``
  and ``jonker_compact_core.h`` compiled by ``oracle/Makefile`` (absent where
  the reference was never checked out and nothing prebuilt travelled along).

Error codes follow ``jv_oracle.c``: 1 = NaN in the input, 2 = -inf.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_ORACLE_SO = _HERE / "libjv_oracle.so"
_REF_SO = _HERE / "_ref" / "libjv_ref.so"

_I64P = ctypes.POINTER(ctypes.c_int64)
_F32P = ctypes.POINTER(ctypes.c_float)

_lib_cache: dict[str, ctypes.CDLL] = {}


class OracleError(RuntimeError):
    """Raised for the reference's rejected inputs (NaN / -inf)."""


def _load(path: Path) -> ctypes.CDLL:
    key = str(path)
    if key not in _lib_cache:
        if not path.exists():
            raise FileNotFoundError(
                f"{path} is not built; run `make -C {_HERE}` (or __graft_entry__.build())"
            )
        lib = ctypes.CDLL(key)
        _lib_cache[key] = lib
    return _lib_cache[key]


def oracle_lib() -> ctypes.CDLL:
    lib = _load(_ORACLE_SO)
    lib.jvo_dense_batch.argtypes = [
        _F32P, ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, _I64P, ctypes.c_int,
    ]
    lib.jvo_dense_batch.restype = ctypes.c_int
    lib.jvo_dense_batch_counted.argtypes = [
        _F32P, ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, _I64P, _I64P,
    ]
    lib.jvo_dense_batch_counted.restype = ctypes.c_int
    lib.jvo_sap_batch_counted.argtypes = lib.jvo_dense_batch_counted.argtypes
    lib.jvo_dense_batch_steps.argtypes = lib.jvo_dense_batch_counted.argtypes
    lib.jvo_dense_batch_steps.restype = ctypes.c_int
    lib.jvo_sap_batch_counted.restype = ctypes.c_int
    lib.jvo_compact_batch.argtypes = lib.jvo_dense_batch.argtypes
    lib.jvo_compact_batch.restype = ctypes.c_int
    lib.jvo_sentinel.argtypes = [_F32P, ctypes.c_int64, ctypes.c_int32, _F32P]
    lib.jvo_sentinel.restype = ctypes.c_int
    return lib


def ref_available() -> bool:
    return _REF_SO.exists()


def ref_lib() -> ctypes.CDLL:
    lib = _load(_REF_SO)
    lib.ref_jv_dense_batch_f32.argtypes = [
        _F32P, ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, _I64P, ctypes.c_int,
    ]
    lib.ref_jv_dense_batch_f32.restype = ctypes.c_int
    lib.ref_jv_compact_batch_f32.argtypes = lib.ref_jv_dense_batch_f32.argtypes
    lib.ref_jv_compact_batch_f32.restype = ctypes.c_int
    return lib


def _prep(costs) -> np.ndarray:
    arr = np.ascontiguousarray(np.asarray(costs, dtype=np.float32))
    if arr.ndim != 3:
        raise ValueError(f"costs must be 3-D (B, N, M), got shape {arr.shape}")
    return arr


def _raise(rc: int) -> None:
    if rc == 1:
        raise OracleError("jonker: cost matrix contains NaN")
    if rc == 2:
        raise OracleError("jonker: cost matrix contains -inf")
    if rc != 0:
        raise OracleError(f"jonker oracle failed with code {rc}")


def jv_dense_batch(costs, threads: int = 0) -> np.ndarray:
    """Oracle ``jonker_dense_batch``: (B, N, M) float32 -> (B, N) int64."""
    arr = _prep(costs)
    b, n, m = arr.shape
    out = np.empty((b, n), dtype=np.int64)
    rc = oracle_lib().jvo_dense_batch(
        arr.ctypes.data_as(_F32P), b, n, m, out.ctypes.data_as(_I64P), threads
    )
    _raise(rc)
    return out


def jv_compact_batch(costs, threads: int = 0) -> np.ndarray:
    """Oracle ``jonker_compact_batch``: (B, N, M) float32 -> (B, N) int64."""
    arr = _prep(costs)
    b, n, m = arr.shape
    out = np.empty((b, n), dtype=np.int64)
    rc = oracle_lib().jvo_compact_batch(
        arr.ctypes.data_as(_F32P), b, n, m, out.ctypes.data_as(_I64P), threads
    )
    _raise(rc)
    return out


def jv_dense_batch_counted(costs) -> tuple[np.ndarray, np.ndarray]:
    """Single-threaded oracle run that also returns per-problem work counts.

    The counts array is (B, 3) int64: reduced-cost evaluations
    ("relaxations"), augmenting paths searched, rows scanned in those paths.
    """
    arr = _prep(costs)
    b, n, m = arr.shape
    out = np.empty((b, n), dtype=np.int64)
    counts = np.zeros((max(b, 1), 3), dtype=np.int64)
    rc = oracle_lib().jvo_dense_batch_counted(
        arr.ctypes.data_as(_F32P), b, n, m, out.ctypes.data_as(_I64P),
        counts.ctypes.data_as(_I64P),
    )
    _raise(rc)
    return out, counts[:b]


def jv_dense_batch_steps(costs) -> tuple[np.ndarray, np.ndarray]:
    """Single-threaded oracle run that also returns the reference order's
    sequential steps per problem, (B, 3) int64: augmenting row reduction steps,
    augmenting paths, rows scanned in the paths' searches."""
    arr = _prep(costs)
    b, n, m = arr.shape
    out = np.empty((b, n), dtype=np.int64)
    steps = np.zeros((max(b, 1), 3), dtype=np.int64)
    rc = oracle_lib().jvo_dense_batch_steps(
        arr.ctypes.data_as(_F32P), b, n, m, out.ctypes.data_as(_I64P),
        steps.ctypes.data_as(_I64P),
    )
    _raise(rc)
    return out, steps[:b]


def sap_batch_counted(costs) -> tuple[np.ndarray, np.ndarray]:
    """Work model of the device's certified path (column reduction, then
    shortest augmenting paths, no row reduction): mapping and per-problem
    counts (B, 3) as :func:`jv_dense_batch_counted`.  Not a reference
    function; its scanned rows + paths are the path's sequential steps."""
    arr = _prep(costs)
    b, n, m = arr.shape
    out = np.empty((b, n), dtype=np.int64)
    counts = np.zeros((max(b, 1), 3), dtype=np.int64)
    rc = oracle_lib().jvo_sap_batch_counted(
        arr.ctypes.data_as(_F32P), b, n, m, out.ctypes.data_as(_I64P),
        counts.ctypes.data_as(_I64P),
    )
    _raise(rc)
    return out, counts[:b]


def sentinel(costs) -> float:
    arr = _prep(costs)
    b, n, m = arr.shape
    val = ctypes.c_float(0.0)
    rc = oracle_lib().jvo_sentinel(
        arr.ctypes.data_as(_F32P), arr.size, max(n, m), ctypes.byref(val)
    )
    _raise(rc)
    return float(np.float32(val.value))


def ref_jv_dense_batch(costs, threads: int = 0) -> np.ndarray:
    """The reference core (compiled from its own source) behind the batch driver."""
    arr = _prep(costs)
    b, n, m = arr.shape
    out = np.empty((b, n), dtype=np.int64)
    rc = ref_lib().ref_jv_dense_batch_f32(
        arr.ctypes.data_as(_F32P), b, n, m, out.ctypes.data_as(_I64P), threads
    )
    _raise(rc)
    return out


def ref_jv_compact_batch(costs, threads: int = 0) -> np.ndarray:
    """The reference's compact solver (header compiled from its own source)
    behind the same batch driver."""
    arr = _prep(costs)
    b, n, m = arr.shape
    out = np.empty((b, n), dtype=np.int64)
    rc = ref_lib().ref_jv_compact_batch_f32(
        arr.ctypes.data_as(_F32P), b, n, m, out.ctypes.data_as(_I64P), threads
    )
    _raise(rc)
    return out


def default_threads() -> int:
    return len(os.sched_getaffinity(0))


def unpack_packed(packed, m: int):
    """The reference CPU op's unpack of packed (B, N) mappings into
    (matches (B, N, 2), unmatched_rows (B, N), unmatched_cols (B, M),
    n_matches (B,)), -1 padded -- a plain-loop restatement of
    assignment/cpu/ops.cpp:387-414 (solve_batch_unpacked)."""
    packed = np.asarray(packed, dtype=np.int64)
    b, n = packed.shape
    matches = np.full((b, n, 2), -1, dtype=np.int64)
    ur = np.full((b, n), -1, dtype=np.int64)
    uc = np.full((b, m), -1, dtype=np.int64)
    nm = np.zeros(b, dtype=np.int64)
    for k in range(b):
        used = [False] * m
        cnt = nur = 0
        for i in range(n):
            j = int(packed[k, i])
            if 0 <= j < m:
                matches[k, cnt] = (i, j)
                cnt += 1
                used[j] = True
            else:
                ur[k, nur] = i
                nur += 1
        nm[k] = cnt
        nuc = 0
        for j in range(m):
            if not used[j]:
                uc[k, nuc] = j
                nuc += 1
    return matches, ur, uc, nm
