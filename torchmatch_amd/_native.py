"""ctypes binding of the C ABI (``include/torchmatch_amd.h``).

The torch ops in ``_C.so`` are the normal way in; this module exposes the
same library to callers that hold raw device pointers (and to the tests,
which exercise the ABI directly).  Loading it needs no GPU.
"""

from __future__ import annotations

import ctypes
from functools import lru_cache

from torchmatch_amd._loader import CABI_SO, ExtensionMissingError

TM_OK = 0
TM_ERR_INVALID_ARGUMENT = 1
TM_ERR_UNSUPPORTED_SHAPE = 2
TM_ERR_WORKSPACE = 3
TM_ERR_LAUNCH = 4
TM_ERR_NAN = 5
TM_ERR_NEG_INF = 6
TM_ERR_HIP = 7
TM_ERR_INTERNAL = 8

TM_JV_FLAG_NAN = 1
TM_JV_FLAG_NEG_INF = 2
TM_JV_FLAG_POS_INF = 4
TM_JV_FLAG_ANY_FINITE = 8
TM_JV_FLAG_NEG_ZERO = 16
TM_JV_FLAG_DONE = 0x80000000

# symbol -> (restype, argtypes); the declarations of include/torchmatch_amd.h
_VP = ctypes.c_void_p
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "tm_jv_max_k": (ctypes.c_int32, []),
    "tm_jv_workspace_bytes": (ctypes.c_size_t, [ctypes.c_int64, ctypes.c_int32, ctypes.c_int32]),
    "tm_jv_workspace_bytes_prefill": (
        ctypes.c_size_t,
        [ctypes.c_int64, ctypes.c_int32, ctypes.c_int32],
    ),
    "tm_jv_dense_batch_f32": (
        ctypes.c_int,
        [_VP, ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, _VP, _VP, ctypes.c_size_t, _VP, _VP],
    ),
    "tm_jv_dense_batch_f32_sync": (
        ctypes.c_int,
        [_VP, ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, _VP, _VP, ctypes.c_size_t,
         ctypes.POINTER(ctypes.c_uint32), _VP],
    ),
    "tm_jv_compact_batch_f32_sync": (
        ctypes.c_int,
        [_VP, ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, _VP, _VP, ctypes.c_size_t,
         ctypes.POINTER(ctypes.c_uint32), _VP],
    ),
    "tm_jv_dense_batch_f32_noalloc": (
        ctypes.c_int, [_VP, ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, _VP, _VP, _VP]
    ),
    "tm_jv_noalloc_scratch_bytes": (ctypes.c_size_t, []),
    "tm_jv_compact_max_k": (ctypes.c_int32, []),
    "tm_jv_compact_batch_f32": (
        ctypes.c_int,
        [_VP, ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, _VP, _VP, ctypes.c_size_t, _VP, _VP],
    ),
    "tm_jv_check_status": (ctypes.c_int, [_VP, _VP]),
    "tm_jv_read_replays": (ctypes.c_int, [_VP, ctypes.POINTER(ctypes.c_uint32), _VP]),
    "tm_jv_status_code": (ctypes.c_int, [_VP]),
    "tm_jv_unpack_i64": (
        ctypes.c_int,
        [_VP, ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, _VP, _VP, _VP, _VP, _VP],
    ),
    "tm_sinkhorn_workspace_bytes": (
        ctypes.c_size_t, [ctypes.c_int64, ctypes.c_int64, ctypes.c_int64]
    ),
    "tm_sinkhorn_prepare_f32": (
        ctypes.c_int,
        [
            _VP, _VP, _VP, _VP, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
            ctypes.c_float, _VP, ctypes.c_size_t, _VP,
        ],
    ),
    "tm_sinkhorn_read_stats": (
        ctypes.c_int,
        [
            _VP, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
            ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(ctypes.c_float), _VP,
        ],
    ),
    "tm_sinkhorn_iterate_f32": (
        ctypes.c_int,
        [
            _VP, _VP, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
            ctypes.POINTER(ctypes.c_double), ctypes.c_int32, ctypes.c_double, ctypes.c_float,
            _VP, _VP, _VP, _VP, ctypes.c_size_t, _VP,
        ],
    ),
    "tm_sinkhorn_f32": (
        ctypes.c_int,
        [
            _VP, _VP, _VP, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
            ctypes.POINTER(ctypes.c_double), ctypes.c_int32, ctypes.c_double,
            _VP, _VP, _VP, _VP, ctypes.c_size_t, _VP,
        ],
    ),
    "tm_sinkhorn_f64_workspace_bytes": (
        ctypes.c_size_t, [ctypes.c_int64, ctypes.c_int64, ctypes.c_int64]
    ),
    "tm_sinkhorn_f64": (
        ctypes.c_int,
        [
            _VP, _VP, _VP, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
            ctypes.POINTER(ctypes.c_double), ctypes.c_int32, ctypes.c_double,
            _VP, _VP, _VP, _VP, ctypes.c_size_t, _VP,
        ],
    ),
}


@lru_cache(maxsize=1)
def lib() -> ctypes.CDLL:
    if not CABI_SO.exists():
        msg = f"{CABI_SO} is not built; run `python torchmatch_amd/_build.py`"
        raise ExtensionMissingError(msg)
    handle = ctypes.CDLL(str(CABI_SO))
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = restype
        fn.argtypes = argtypes
    return handle


def jv_max_k() -> int:
    return int(lib().tm_jv_max_k())
