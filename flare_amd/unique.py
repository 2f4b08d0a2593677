"""First-occurrence dedup on the GPU (``src/flare/ops/sparse_unique.py:52-77``).

Same contract: ``(unique, inverse:int32, first_indices:int64)`` with unique
keys in the order of their first occurrence; empty input returns
``(values.copy(), int32[0], int64[0])``; non-integer keys raise ``TypeError``.
numpy input returns numpy arrays (computed on the GPU, copied back); torch or
other DLPack device input returns device tensors.  The algorithm is a stable
radix sort of (key, position) pairs, segment heads, and a scan of
"first occurrence" flags in input order (``flare_amd/csrc/backward.hip``).
"""

from __future__ import annotations

from typing import Any

import numpy as np
import torch

from flare_amd import _native
from flare_amd.conversion import contiguous, key_code, to_device

_NUMPY_KEYS = {np.dtype(np.int32), np.dtype(np.int64), np.dtype(np.uint32), np.dtype(np.uint64)}


def unique_first_occurrence(values: Any, *, key_bound: int = 0, stream: Any = None):
    """Deduplicate integer keys in first-occurrence order on the current GPU.

    ``key_bound > 0`` promises ``0 <= key < key_bound`` and saves one
    device-to-host read of the key range.  The unique count is read back once.
    """
    host = isinstance(values, np.ndarray) or not hasattr(values, "__dlpack__") and not isinstance(values, torch.Tensor)
    if host:
        arr = np.asarray(values)
        if arr.ndim != 1:
            arr = arr.reshape(-1)
        if arr.dtype.kind not in "iu":
            raise TypeError(f"sparse unique requires integer keys, got {arr.dtype}")
        if arr.dtype not in _NUMPY_KEYS:
            arr = arr.astype(np.int64 if arr.dtype.kind == "i" else np.uint64)
        if arr.size == 0:
            return arr.copy(), np.empty(0, np.int32), np.empty(0, np.int64)
        unique, inverse, first = _unique_device(torch.from_numpy(np.ascontiguousarray(arr)), key_bound, stream)
        return unique.cpu().numpy(), inverse.cpu().numpy(), first.cpu().numpy()
    tensor = values if isinstance(values, torch.Tensor) else torch.from_dlpack(values)
    if tensor.dtype.is_floating_point or tensor.dtype.is_complex or tensor.dtype == torch.bool:
        raise TypeError(f"sparse unique requires integer keys, got {tensor.dtype}")
    return _unique_device(tensor.reshape(-1), key_bound, stream)


def _unique_device(tensor: torch.Tensor, key_bound: int, stream: Any):
    device = torch.device("cuda", torch.cuda.current_device()) if tensor.device.type != "cuda" else tensor.device
    if tensor.dtype in (torch.int8, torch.int16, torch.uint8, torch.uint16):
        tensor = tensor.to(torch.int32)
    code = key_code(tensor.dtype)
    if code is None:
        raise TypeError(f"sparse unique requires integer keys, got {tensor.dtype}")
    s = torch.cuda.current_stream(device) if stream is None else stream
    with torch.cuda.stream(s):
        keys = contiguous(to_device(tensor, device))
        n = int(keys.numel())
        if n == 0:
            return keys.clone(), torch.empty(0, dtype=torch.int32, device=device), torch.empty(0, dtype=torch.int64, device=device)
        unique = torch.empty(n, dtype=keys.dtype, device=device)
        inverse = torch.empty(n, dtype=torch.int32, device=device)
        first = torch.empty(n, dtype=torch.int64, device=device)
        count = torch.empty(1, dtype=torch.int64, device=device)
        nbytes = _native.library().flare_unique_workspace_bytes(n, code)
        workspace = torch.empty(nbytes, dtype=torch.uint8, device=device)
        _native.call(
            "flare_unique_first_occurrence", keys.data_ptr(), code, n, int(key_bound),
            unique.data_ptr(), inverse.data_ptr(), first.data_ptr(), count.data_ptr(),
            workspace.data_ptr(), nbytes, int(s.cuda_stream),
        )
        u = int(count.item())
    return unique[:u], inverse, first[:u]
