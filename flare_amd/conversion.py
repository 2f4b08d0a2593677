"""Buffer exchange for the HIP path: DLPack (producers or capsules) in, device arrays out.

Device arrays are imported zero-copy (``torch.from_dlpack``); host arrays are
copied to the device on the operator's stream.  This mirrors
``src/flare/kernels/conversion.py:97-127`` and ``gpu_cupy.py:301-319``, which
know CUDA (DLPack device type 2) and CPU (1); on ROCm the device type is
kDLROCM (10), accepted here alongside 2.
"""

from __future__ import annotations

from typing import Any

import numpy as np
import torch

from flare_amd import _native

DLPACK_DEVICE_CPU = 1
DLPACK_DEVICE_CUDA = 2
DLPACK_DEVICE_ROCM = 10

_STORAGE_CODES = {
    torch.float32: _native.FLOAT32,
    torch.float16: _native.FLOAT16,
    torch.bfloat16: _native.BFLOAT16,
}
_KEY_CODES = {
    torch.int32: _native.INT32,
    torch.int64: _native.INT64,
    torch.uint32: _native.UINT32,
    torch.uint64: _native.UINT64,
}
TORCH_VALUE_DTYPES = {"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16}


def storage_code(dtype: torch.dtype) -> int | None:
    return _STORAGE_CODES.get(dtype)


def key_code(dtype: torch.dtype) -> int | None:
    return _KEY_CODES.get(dtype)


def dtype_name(dtype: torch.dtype) -> str:
    return str(dtype).replace("torch.", "")


def is_dlpack_capsule(value: Any) -> bool:
    """A legacy DLPack ``PyCapsule`` (named "dltensor"), as ``to_dlpack`` and the
    reference's ``prepare_dlpack_input`` produce (``dynamic_embedding.py:396-400,514``)."""
    return type(value).__name__ == "PyCapsule"


def to_device(value: Any, device: torch.device, *, non_blocking: bool = True) -> torch.Tensor:
    """Import ``value`` as a torch tensor on ``device`` (caller enters the stream).

    Accepts torch tensors, ``DeviceArray``s, DLPack producers (device types 1,
    2 and 10), legacy DLPack capsules (consumed: a capsule imports once),
    objects exposing ``__cuda_array_interface__``, and numpy arrays /
    array-likes.  Raises ``TypeError`` for anything else.
    """
    from flare_amd.array import DeviceArray

    if isinstance(value, torch.Tensor):
        tensor = value
    elif isinstance(value, DeviceArray):
        tensor = value.tensor
    elif isinstance(value, np.ndarray):
        tensor = torch.from_numpy(np.ascontiguousarray(value))
    elif is_dlpack_capsule(value):
        tensor = torch.from_dlpack(value)
    elif hasattr(value, "__cuda_array_interface__") and not hasattr(value, "__dlpack__"):
        tensor = torch.as_tensor(value, device=device)
    elif hasattr(value, "__dlpack__"):
        if not hasattr(value, "__dlpack_device__"):
            raise TypeError(
                "DLPack conversion requires __dlpack_device__ to identify the source device, "
                f"got {type(value).__name__}."
            )
        device_type, _ = value.__dlpack_device__()
        if device_type not in (DLPACK_DEVICE_CPU, DLPACK_DEVICE_CUDA, DLPACK_DEVICE_ROCM):
            raise TypeError(
                f"unsupported DLPack device type {device_type!r} from {type(value).__name__}"
            )
        tensor = torch.from_dlpack(value)
    elif isinstance(value, (list, tuple)) or np.isscalar(value):
        tensor = torch.from_numpy(np.ascontiguousarray(np.asarray(value)))
    else:
        raise TypeError(
            f"Value of type {type(value).__name__} does not support the DLPack protocol or the array interface."
        )
    if tensor.device != device:
        tensor = tensor.to(device, non_blocking=non_blocking and tensor.device.type == "cpu" and tensor.is_pinned())
    return tensor


def contiguous(tensor: torch.Tensor) -> torch.Tensor:
    return tensor if tensor.is_contiguous() else tensor.contiguous()


def ptr(tensor: torch.Tensor | None) -> int | None:
    return None if tensor is None else tensor.data_ptr()
