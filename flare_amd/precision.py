"""dtype contract of the sparse path (``src/flare/runtime/sparse_precision.py:8-49``).

Same whitelists, same ``ValueError`` text, with one documented extension:
``bfloat16`` is accepted as a *value* (storage) dtype, which the reference
rejects (``sparse_precision.py:11``); accumulation and optimizer state stay
float32.
"""

from __future__ import annotations

from typing import Any

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


def prepare_sparse_native_gradient(values: Any, *, transport_dtype: str, native_dtype: str,
                                   validate_values: bool = False) -> Any:
    """Transport (bf16/fp32) -> native fp32 gradient (``sparse_precision.py:150-192``).

    Accepts torch tensors (device or host).  Raises ``TypeError`` on a dtype
    mismatch and ``FloatingPointError`` on non-finite values when
    ``validate_values`` is set.
    """
    import torch

    require_sparse_gradient_transport_dtype(transport_dtype)
    require_sparse_gradient_dtype(native_dtype)
    if not isinstance(values, torch.Tensor):
        raise TypeError(f"unsupported sparse gradient tensor type: {type(values).__name__}")
    expected = {"bfloat16": torch.bfloat16, "float32": torch.float32}[transport_dtype]
    if values.dtype != expected:
        raise TypeError(
            f"sparse gradient transport dtype mismatch: expected={transport_dtype} "
            f"actual={str(values.dtype).replace('torch.', '')}"
        )
    if not isinstance(validate_values, bool):
        raise TypeError("validate_values must be bool")
    cast = values.to(dtype=torch.float32)
    if validate_values and not bool(torch.isfinite(cast).all()):
        raise FloatingPointError("non-finite sparse values at sparse_native_gradient")
    return cast
