"""Device arrays at the operator and store boundary.

The reference's GPU backend hands its callers CuPy arrays
(``src/flare/kernels/backends/gpu_cupy.py:301-330``), and the unchanged callers
rely on that array protocol:

* ``np.dtype(grad.dtype).name`` and ``grad.astype(transport)`` on the
  ``scatter_pooled`` result (``recipes/recsys/ranking/workers/train_worker.py:518-522``);
* ``prepare_sparse_native_gradient`` routes arrays that expose
  ``__cuda_array_interface__`` to ``values.astype(dtype, copy=False)``
  (``src/flare/runtime/sparse_precision.py:179-180``);
* ``int(valid_count_device[0])``, ``.shape``, ``.ndim``
  (``recipes/recsys/ranking/schema/materialization.py:41-53``);
* DLPack export to JAX (``to_jax_array_with_lease``, ``train_worker.py:298-330``).

``DeviceArray`` is that protocol over a torch tensor in HBM: numpy dtypes,
``astype`` (floating-point casts run on this library's HIP conversion kernel,
rounding to nearest even), ``__cuda_array_interface__`` (version 3, the HIP
device pointer), ``__dlpack__`` / ``__dlpack_device__`` (DLPack device type 10,
ROCm), and host copies through ``get()`` / ``__array__``.  bfloat16 maps to
``ml_dtypes.bfloat16`` where that package is installed (JAX ships it) and to
a named placeholder dtype otherwise.
"""

from __future__ import annotations

from typing import Any

import numpy as np
import torch

from flare_amd import _native

try:  # the numpy bfloat16 type JAX uses; absent in plain numpy installs
    import ml_dtypes as _ml_dtypes  # type: ignore

    _NP_BFLOAT16: Any = np.dtype(_ml_dtypes.bfloat16)
except ImportError:  # pragma: no cover - depends on the environment
    _NP_BFLOAT16 = None


class BFloat16DType:
    """Stands in for numpy's missing bfloat16 dtype: compares equal to ``"bfloat16"``."""

    name = "bfloat16"
    itemsize = 2
    kind = "V"
    str = "<V2"

    def __eq__(self, other: Any) -> bool:
        if isinstance(other, BFloat16DType):
            return True
        if isinstance(other, str):
            return other == "bfloat16"
        return getattr(other, "name", None) == "bfloat16"

    def __hash__(self) -> int:
        return hash("bfloat16")

    def __repr__(self) -> str:
        return "dtype('bfloat16')"


BFLOAT16 = BFloat16DType()

_TORCH_OF_NAME = {
    "float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16,
    "float64": torch.float64, "int8": torch.int8, "uint8": torch.uint8, "int16": torch.int16,
    "int32": torch.int32, "int64": torch.int64, "uint32": torch.uint32, "uint64": torch.uint64,
    "bool": torch.bool,
}
_NAME_OF_TORCH = {v: k for k, v in _TORCH_OF_NAME.items()}
_FLOAT_CODES = {torch.float32: _native.FLOAT32, torch.float16: _native.FLOAT16, torch.bfloat16: _native.BFLOAT16}


def dtype_name(dtype: Any) -> str:
    """Name of a numpy / torch / string dtype ("float32", "bfloat16", ...)."""
    if isinstance(dtype, torch.dtype):
        return _NAME_OF_TORCH[dtype]
    if isinstance(dtype, str):
        return "bfloat16" if dtype == "bfloat16" else np.dtype(dtype).name
    name = getattr(dtype, "name", None)
    if name == "bfloat16":
        return name
    return np.dtype(dtype).name


def torch_dtype(dtype: Any) -> torch.dtype:
    try:
        return _TORCH_OF_NAME[dtype_name(dtype)]
    except KeyError as error:
        raise TypeError(f"unsupported device array dtype {dtype!r}") from error


def numpy_dtype(dtype: torch.dtype) -> Any:
    if dtype == torch.bfloat16:
        return _NP_BFLOAT16 if _NP_BFLOAT16 is not None else BFLOAT16
    return np.dtype(_NAME_OF_TORCH[dtype])


def _typestr(dtype: torch.dtype) -> str:
    if dtype == torch.bfloat16:
        return "<V2"
    return np.dtype(_NAME_OF_TORCH[dtype]).str


def convert(src: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """``src`` cast to ``dtype`` on the device, on the current stream.

    float32 / float16 / bfloat16 to one another: this library's conversion
    kernel (``flare_convert``), round to nearest even.  Integer and other casts
    are PyTorch's element-wise copies.
    """
    if src.dtype == dtype:
        return src
    src = src if src.is_contiguous() else src.contiguous()
    if src.device.type == "cuda" and src.dtype in _FLOAT_CODES and dtype in _FLOAT_CODES:
        out = torch.empty(src.shape, dtype=dtype, device=src.device)
        if src.numel():
            _native.call("flare_convert", src.data_ptr(), _FLOAT_CODES[src.dtype], out.data_ptr(),
                         _FLOAT_CODES[dtype], src.numel(), int(torch.cuda.current_stream(src.device).cuda_stream))
        return out
    return src.to(dtype)


class DeviceArray:
    """A CuPy-style view of a device tensor (see the module docstring)."""

    __slots__ = ("_tensor",)
    __array_priority__ = 100

    def __init__(self, tensor: torch.Tensor):
        if isinstance(tensor, DeviceArray):
            tensor = tensor.tensor
        if not isinstance(tensor, torch.Tensor):
            raise TypeError(f"DeviceArray wraps a torch tensor, got {type(tensor).__name__}")
        self._tensor = tensor

    # -- the tensor and its metadata ------------------------------------------------
    @property
    def tensor(self) -> torch.Tensor:
        return self._tensor

    @property
    def dtype(self) -> Any:
        return numpy_dtype(self._tensor.dtype)

    @property
    def shape(self) -> tuple[int, ...]:
        return tuple(self._tensor.shape)

    @property
    def ndim(self) -> int:
        return self._tensor.dim()

    @property
    def size(self) -> int:
        return self._tensor.numel()

    @property
    def itemsize(self) -> int:
        return self._tensor.element_size()

    @property
    def nbytes(self) -> int:
        return self._tensor.numel() * self._tensor.element_size()

    @property
    def strides(self) -> tuple[int, ...]:
        return tuple(s * self._tensor.element_size() for s in self._tensor.stride())

    @property
    def device(self) -> torch.device:
        return self._tensor.device

    def data_ptr(self) -> int:
        return self._tensor.data_ptr()

    def __len__(self) -> int:
        if self._tensor.dim() == 0:
            raise TypeError("len() of a 0-d device array")
        return int(self._tensor.shape[0])

    def __repr__(self) -> str:
        return f"DeviceArray(shape={self.shape}, dtype={dtype_name(self._tensor.dtype)}, device={self._tensor.device})"

    # -- views and casts ----------------------------------------------------------------
    def reshape(self, *shape: Any) -> "DeviceArray":
        if len(shape) == 1 and isinstance(shape[0], (tuple, list)):
            shape = tuple(shape[0])
        return DeviceArray(self._tensor.reshape(*shape))

    def ravel(self) -> "DeviceArray":
        return DeviceArray(self._tensor.reshape(-1))

    def __getitem__(self, key: Any) -> "DeviceArray":
        if isinstance(key, DeviceArray):
            key = key.tensor
        return DeviceArray(self._tensor[key])

    def astype(self, dtype: Any, copy: bool = True) -> "DeviceArray":
        target = torch_dtype(dtype)
        if target == self._tensor.dtype:
            return DeviceArray(self._tensor.clone()) if copy else self
        return DeviceArray(convert(self._tensor, target))

    def copy(self) -> "DeviceArray":
        return DeviceArray(self._tensor.clone())

    # -- scalars --------------------------------------------------------------------------
    def item(self) -> Any:
        return self._tensor.item()

    def __int__(self) -> int:
        return int(self._tensor.item())

    def __float__(self) -> float:
        return float(self._tensor.item())

    def __index__(self) -> int:
        if self._tensor.dtype.is_floating_point:
            raise TypeError("only integer device arrays can be used as an index")
        return int(self._tensor.item())

    def __bool__(self) -> bool:
        return bool(self._tensor.item())

    # -- host copies ------------------------------------------------------------------------
    def get(self, stream: Any = None) -> np.ndarray:
        """Host copy (blocking), as ``cupy.ndarray.get``; bfloat16 needs ``ml_dtypes``."""
        t = self._tensor
        if t.dtype == torch.bfloat16:
            if _NP_BFLOAT16 is None:
                raise TypeError("a host copy of a bfloat16 device array needs ml_dtypes")
            return t.view(torch.int16).cpu().numpy().view(_NP_BFLOAT16)
        return t.detach().cpu().numpy()

    def __array__(self, dtype: Any = None, copy: Any = None) -> np.ndarray:
        host = self.get()
        return host if dtype is None else host.astype(dtype)

    # -- zero-copy exchange ---------------------------------------------------------------
    @property
    def __cuda_array_interface__(self) -> dict:
        t = self._tensor
        if t.device.type != "cuda":
            raise AttributeError("__cuda_array_interface__ is defined for device arrays only")
        return {
            "shape": tuple(t.shape),
            "typestr": _typestr(t.dtype),
            "data": (t.data_ptr(), False),
            "version": 3,
            "strides": None if t.is_contiguous() else self.strides,
            "stream": None,
        }

    def __dlpack__(self, *args: Any, **kwargs: Any) -> Any:
        return self._tensor.__dlpack__(*args, **kwargs)

    def __dlpack_device__(self) -> tuple:
        return self._tensor.__dlpack_device__()


def as_device_array(value: Any) -> DeviceArray:
    return value if isinstance(value, DeviceArray) else DeviceArray(value)
