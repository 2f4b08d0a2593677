"""ctypes binding of ``libflare_amd.so`` (declared in ``include/flare_amd.h``).

There is no fallback: if the library is missing or a call fails, a Python
exception is raised.  Status codes map onto the exception classes the
reference raises at the same boundaries
(``src/flare/kernels/backends/gpu_cupy.py:351-354,398-401,479-483``).
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIBRARY_PATH = Path(__file__).resolve().parent / "libflare_amd.so"

# flare_status
OK, ERR_DTYPE, ERR_SHAPE, ERR_WIDTH, ERR_ARGUMENT, ERR_WORKSPACE, ERR_HIP, ERR_LIMIT = range(8)
# flare_dtype
FLOAT32, FLOAT16, BFLOAT16, INT32, INT64, UINT32, UINT64 = range(7)
# flare_pooling
POOL_SUM, POOL_MEAN, POOL_WEIGHTED = range(3)
# flare_layout
LAYOUT_SAMPLE_MAJOR, LAYOUT_TABLE_MAJOR = range(2)
LAYOUT_ONE_ID_PER_BAG = 0x100  # flag for the dedup: every bag holds exactly one id
# flare_optimizer_kind
OPT_NONE, OPT_SGD, OPT_ADAM, OPT_ROWWISE_ADAGRAD = range(4)

# device error bits
ERR_BIT_INDEX = 1
ERR_BIT_SPIN = 2


class FlareOptimizer(ctypes.Structure):
    _fields_ = [
        ("kind", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
        ("learning_rate", ctypes.c_double),
        ("beta1", ctypes.c_double),
        ("beta2", ctypes.c_double),
        ("eps", ctypes.c_double),
        ("weight_decay", ctypes.c_double),
    ]


_vp = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_sz = ctypes.c_size_t

# name -> (restype, argtypes)
SIGNATURES = {
    "flare_last_error": (ctypes.c_char_p, []),
    "flare_abi_version": (_i32, []),
    "flare_gather": (_i32, [_vp, _i32, _i64, _i32, _vp, _i64, _i32, _vp, _vp]),
    "flare_gather_pooled": (_i32, [_vp, _i32, _i64, _i32, _vp, _i64, _i32, _i32, _i32, _i32, _vp, _vp, _vp]),
    "flare_gather_pooled_csr": (_i32, [_vp, _i32, _i64, _i32, _vp, _i32, _i64, _vp, _i32, _i64, _vp, _i32, _i32, _vp, _vp, _vp]),
    "flare_scatter_workspace_bytes": (_sz, [_i64, _i64, _i32]),
    "flare_scatter": (_i32, [_i64, _i32, _vp, _i64, _i32, _vp, _vp, _vp, _sz, _vp]),
    "flare_scatter_pooled": (_i32, [_i64, _i32, _vp, _i64, _i32, _vp, _i64, _i32, _i32, _vp, _vp, _sz, _vp]),
    "flare_scatter_ex": (_i32, [_i64, _i32, _vp, _i64, _i32, _vp, _vp, _i32, _vp, _sz, _vp]),
    "flare_scatter_pooled_ex": (_i32, [_i64, _i32, _vp, _i64, _i32, _vp, _i64, _i32, _i32, _vp, _i32, _vp, _sz, _vp]),
    "flare_unique_workspace_bytes": (_sz, [_i64, _i32]),
    "flare_unique_first_occurrence": (_i32, [_vp, _i32, _i64, _i64, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "flare_unique_first_occurrence_noalloc": (_i32, [_vp, _i32, _i64, _i64, _vp, _vp, _vp, _vp, _vp]),
    "flare_sparse_update_workspace_bytes": (_sz, [_i64, _i64, _i32]),
    "flare_sparse_update": (_i32, [_vp, _i32, _i64, _i32, _vp, _vp, _vp, ctypes.POINTER(FlareOptimizer), _vp, _i64, _vp, _i32, _vp, _sz, _vp]),
    "flare_pooled_backward_workspace_bytes": (_sz, [_i64, _i64, _i32]),
    "flare_pooled_backward": (_i32, [_vp, _i32, _i64, _i32, _vp, _vp, _vp, ctypes.POINTER(FlareOptimizer), _vp, _i32, _i64, _vp, _i32, _i64, _vp, _i32, _i32, _vp, _vp, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "flare_pooled_dedup": (_i32, [_vp, _i32, _i64, _vp, _i32, _i64, _vp, _i64, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _sz, _vp]),
    "flare_pooled_apply": (_i32, [_vp, _i32, _i64, _i32, _vp, _vp, _vp, ctypes.POINTER(FlareOptimizer), _i64, _i32, _i64, _i32, _vp, _vp, _i32, _vp, _vp, _vp, _sz, _vp]),
    "flare_pooled_apply_ex": (_i32, [_vp, _i32, _i64, _i32, _vp, _vp, _vp, ctypes.POINTER(FlareOptimizer), _i64, _i32, _i64, _i32, _vp, _vp, _i32, _i32, _vp, _i32, _vp, _vp, _vp, _sz, _vp]),
    "flare_sparse_update_ex": (_i32, [_vp, _i32, _i64, _i32, _vp, _vp, _vp, ctypes.POINTER(FlareOptimizer), _vp, _i64, _vp, _i32, _i32, _vp, _i32, _vp, _sz, _vp]),
    "flare_check_finite": (_i32, [_vp, _i32, _i64, _vp, _vp]),
    "flare_set_update_events": (_i32, [_vp, _i32]),
    "flare_zero_bytes": (_i32, [_vp, _i64, _vp]),
    "flare_convert": (_i32, [_vp, _i32, _vp, _i32, _i64, _vp]),
    "flare_stream_create": (_i32, [_vp]),
    "flare_stream_synchronize": (_i32, [_vp]),
    "flare_stream_destroy": (_i32, [_vp]),
    "flare_keymap_bytes": (_sz, [_i64]),
    "flare_keymap_init": (_i32, [_vp, _i64, _vp]),
    "flare_keymap_workspace_bytes": (_sz, [_i64]),
    "flare_keymap_lookup_or_insert": (_i32, [_vp, _i64, _vp, _i64, _i32, _vp, _i32, _i64, _i32, ctypes.c_float,
                                             ctypes.c_float, ctypes.c_uint64, _vp, _vp, _vp, _sz, _vp]),
    "flare_keymap_rehash": (_i32, [_vp, _i64, _vp, _i64, _vp]),
    "flare_keymap_export_workspace_bytes": (_sz, [_i64]),
    "flare_keymap_export": (_i32, [_vp, _i64, _vp, _vp, _vp, _vp, _sz, _vp]),
    "flare_copy_rows": (_i32, [_vp, _i64, _vp, _i64, _i64, _vp, _vp, _i64, _vp]),
    "flare_nested_global_positions": (_i32, [_vp, _i64, _i32, _vp, _vp, _vp, _i64, _vp, _vp, _vp]),
    "flare_take_device_errors": (_i32, [_vp]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def library() -> ctypes.CDLL:
    """Load the HIP library once; raise if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIBRARY_PATH.exists():
                raise RuntimeError(
                    f"{LIBRARY_PATH} is missing: build it with `python -m flare_amd.build` "
                    "(the HIP path has no CPU fallback)"
                )
            lib = ctypes.CDLL(str(LIBRARY_PATH))
            for name, (restype, argtypes) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = restype
                fn.argtypes = argtypes
            _lib = lib
    return _lib


def last_error() -> str:
    msg = library().flare_last_error()
    return msg.decode("utf-8", "replace") if msg else ""


def check(status: int) -> None:
    """Raise the exception class matching a flare_status code."""
    if status == OK:
        return
    message = last_error()
    if status == ERR_DTYPE:
        raise TypeError(message)
    if status in (ERR_SHAPE, ERR_WIDTH, ERR_ARGUMENT, ERR_WORKSPACE, ERR_LIMIT):
        raise ValueError(message)
    raise RuntimeError(message or f"flare_amd call failed with status {status}")


def call(name: str, *args) -> None:
    check(getattr(library(), name)(*args))
