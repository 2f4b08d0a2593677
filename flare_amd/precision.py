"""dtype contract of the sparse path (``src/flare/runtime/sparse_precision.py:8-49``).

Same whitelists, same ``ValueError`` text, with one documented extension:
``bfloat16`` is accepted as a *value* (storage) dtype, which the reference
rejects (``sparse_precision.py:11``); accumulation and optimizer state stay
float32.
"""

from __future__ import annotations

from typing import Any

import numpy as np

SPARSE_FLOAT16_DTYPE = "float16"
SPARSE_BFLOAT16_DTYPE = "bfloat16"
SPARSE_FLOAT32_DTYPE = "float32"
SPARSE_VALUE_DTYPES = frozenset({SPARSE_FLOAT16_DTYPE, SPARSE_BFLOAT16_DTYPE, SPARSE_FLOAT32_DTYPE})
SPARSE_GRADIENT_TRANSPORT_DTYPES = frozenset({SPARSE_BFLOAT16_DTYPE, SPARSE_FLOAT32_DTYPE})
SPARSE_GRADIENT_DTYPES = frozenset({SPARSE_FLOAT32_DTYPE})
SPARSE_OPTIMIZER_DTYPES = frozenset({SPARSE_FLOAT32_DTYPE})
SPARSE_NATIVE_GRADIENT_DTYPE = SPARSE_FLOAT32_DTYPE


def _require_dtype(value: Any, allowed: frozenset[str], field: str) -> str:
    if not isinstance(value, str) or value not in allowed:
        raise ValueError(f"{field} must be one of {sorted(allowed)!r}, got {value!r}")
    return value


def require_sparse_value_dtype(value: Any) -> str:
    return _require_dtype(value, SPARSE_VALUE_DTYPES, "sparse embedding value_dtype")


def require_sparse_gradient_dtype(value: Any) -> str:
    return _require_dtype(value, SPARSE_GRADIENT_DTYPES, "sparse embedding gradient_dtype")


def require_sparse_gradient_transport_dtype(value: Any) -> str:
    return _require_dtype(
        value, SPARSE_GRADIENT_TRANSPORT_DTYPES, "sparse embedding gradient_transport_dtype"
    )


def require_sparse_optimizer_dtype(value: Any) -> str:
    return _require_dtype(value, SPARSE_OPTIMIZER_DTYPES, "sparse embedding optimizer_dtype")


SUPPORTED_KEY_DTYPES = frozenset({"int32", "uint32", "int64", "uint64"})


def require_key_dtype(value: Any) -> str:
    if not isinstance(value, str) or value not in SUPPORTED_KEY_DTYPES:
        raise ValueError(
            "sparse embedding key_dtype must be one of "
            f"{tuple(sorted(SUPPORTED_KEY_DTYPES))!r}, got {value!r}"
        )
    return value


def _numpy_dtype_name(values: Any) -> str:
    """dtype name of a numpy / device / torch array (``sparse_precision.py:76-95``)."""
    from flare_amd.array import dtype_name

    try:
        return dtype_name(values.dtype)
    except (AttributeError, KeyError, TypeError) as error:
        raise TypeError(f"unsupported sparse tensor dtype: {getattr(values, 'dtype', None)}") from error


def require_sparse_key_dtype(values: Any, key_dtype: str, *, boundary: str) -> Any:
    """Key array dtype check (``sparse_precision.py:55-73``)."""
    expected = require_key_dtype(key_dtype)
    try:
        actual = _numpy_dtype_name(values)
    except TypeError as error:
        raise TypeError(f"sparse key dtype validation at {boundary} requires an array dtype") from error
    if actual not in SUPPORTED_KEY_DTYPES:
        raise TypeError(
            f"sparse key dtype at {boundary} must be one of {sorted(SUPPORTED_KEY_DTYPES)!r}, got {actual!r}"
        )
    if actual != expected:
        raise TypeError(f"sparse key dtype mismatch at {boundary}: expected={expected}, got={actual}")
    return values


def require_sparse_tensor_dtype(values: Any, dtype: str, *, boundary: str) -> Any:
    """``sparse_precision.py:98-118``: values of exactly ``dtype``."""
    if dtype not in SPARSE_VALUE_DTYPES | SPARSE_GRADIENT_TRANSPORT_DTYPES:
        raise ValueError(
            f"sparse precision check requires float16, bfloat16, or float32, got {dtype!r}"
        )
    actual = _numpy_dtype_name(values)
    if actual != dtype:
        raise TypeError(
            f"sparse precision check dtype mismatch at {boundary}: expected={dtype} actual={actual}"
        )
    return values


def _device_all_finite(tensor: Any) -> bool:
    """One pass of this library's finite-check kernel over a device tensor (synchronizes)."""
    import torch

    from flare_amd import _native
    from flare_amd.conversion import contiguous, storage_code

    t = contiguous(tensor)
    code = storage_code(t.dtype)
    if code is None:
        raise TypeError(f"unsupported sparse precision check tensor dtype: {t.dtype}")
    if t.numel() == 0:
        return True
    flag = torch.empty(1, dtype=torch.int32, device=t.device)
    stream = torch.cuda.current_stream(t.device)
    _native.call("flare_check_finite", t.data_ptr(), code, t.numel(), flag.data_ptr(), int(stream.cuda_stream))
    stream.synchronize()
    return int(flag.item()) == 0


def require_finite_sparse_values(values: Any, dtype: str, *, boundary: str) -> Any:
    """``sparse_precision.py:121-147``: ``FloatingPointError`` on inf / NaN.  Device arrays
    (``DeviceArray`` or torch device tensors) are checked by the HIP finite-check kernel."""
    import torch

    from flare_amd.array import DeviceArray

    require_sparse_tensor_dtype(values, dtype, boundary=boundary)
    if isinstance(values, np.ndarray):
        finite = bool(np.isfinite(values).all())
    elif isinstance(values, DeviceArray) or (isinstance(values, torch.Tensor) and values.device.type == "cuda"):
        finite = _device_all_finite(values.tensor if isinstance(values, DeviceArray) else values)
    elif isinstance(values, torch.Tensor):
        finite = bool(torch.isfinite(values).all())
    else:
        raise TypeError(f"unsupported sparse precision check tensor type: {type(values).__name__}")
    if not finite:
        raise FloatingPointError(f"non-finite sparse values at {boundary}")
    return values


def prepare_sparse_native_gradient(values: Any, *, transport_dtype: str, native_dtype: str,
                                   validate_values: bool = False) -> Any:
    """Transport (bf16/fp32) -> native fp32 gradient (``sparse_precision.py:150-192``).

    Accepts numpy arrays (cast on the host), ``DeviceArray``s (cast by the HIP
    conversion kernel) and torch tensors, as the reference accepts numpy, CuPy
    and torch.  Raises ``TypeError`` on a transport dtype mismatch and
    ``FloatingPointError`` on non-finite values when ``validate_values`` is set.
    """
    import torch

    from flare_amd.array import DeviceArray, convert

    require_sparse_gradient_transport_dtype(transport_dtype)
    require_sparse_gradient_dtype(native_dtype)
    actual = _numpy_dtype_name(values)
    if actual != transport_dtype:
        raise TypeError(
            f"sparse gradient transport dtype mismatch: expected={transport_dtype} actual={actual}"
        )
    if isinstance(values, np.ndarray):
        cast = values.astype(np.dtype(native_dtype), copy=False)
    elif isinstance(values, DeviceArray):
        cast = values.astype(native_dtype, copy=False)
    elif isinstance(values, torch.Tensor):
        cast = convert(values, torch.float32) if values.device.type == "cuda" else values.to(torch.float32)
    else:
        raise TypeError(f"unsupported sparse gradient tensor type: {type(values).__name__}")
    if not isinstance(validate_values, bool):
        raise TypeError("validate_values must be bool")
    if validate_values:
        return require_finite_sparse_values(cast, native_dtype, boundary="sparse_native_gradient")
    return cast
