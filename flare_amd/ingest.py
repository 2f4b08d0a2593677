"""CSR-native ingest helpers on the GPU.

``unique_global_flat_positions`` restates ``_unique_global_flat_positions``
(``src/flare/runtime/fluxway/workers/sparse_input.py:85-113``): the dense global
position of each unique id's first occurrence in a ragged (nested CSR) batch, so the
input worker need not walk the splits on the host.
"""

from __future__ import annotations

import ctypes
from typing import Any, Sequence

import numpy as np
import torch

from flare_amd import _native
from flare_amd.conversion import contiguous, to_device


def unique_global_flat_positions(nested_splits: Sequence[Any], flat_first_indices: Any, widths: Sequence[int],
                                 origin_indices: Any, group_name: str = "", *, device: Any = None,
                                 stream: Any = None):
    """int32 dense positions of ``flat_first_indices`` (see ``flare_nested_global_positions``).

    Raises ``ValueError`` as the reference does when the nesting depth differs from the dense
    widths, and when a path leaves the dense shape (a local row past the origins, or a
    nested index past its width).  Numpy inputs give a numpy result; device inputs a tensor.
    """
    if len(nested_splits) != len(widths):
        raise ValueError(
            f"[InputSPMD._sparse_unique:{group_name}] nested levels "
            f"{len(nested_splits)} != dense widths {len(widths)}."
        )
    host_result = isinstance(flat_first_indices, np.ndarray)
    dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    _native.library()
    s = torch.cuda.current_stream(dev) if stream is None else stream
    caller = torch.cuda.current_stream(dev)
    if s != caller:
        s.wait_stream(caller)  # device inputs the caller's stream is still producing
    with torch.cuda.stream(s):  # the conversions and the kernel on one stream, in order
        splits = [contiguous(to_device(sp, dev).reshape(-1).to(torch.int64)) for sp in nested_splits]
        first = contiguous(to_device(flat_first_indices, dev).reshape(-1).to(torch.int64))
        origin = contiguous(to_device(origin_indices, dev).reshape(-1).to(torch.int64))
        out = torch.empty(max(int(first.numel()), 1), dtype=torch.int32, device=dev)
        levels = len(splits)
        ptrs = (ctypes.c_void_p * levels)(*[sp.data_ptr() for sp in splits])
        lengths = (ctypes.c_int64 * levels)(*[int(sp.numel()) for sp in splits])
        dims = (ctypes.c_int64 * levels)(*[int(w) for w in widths])
        _native.call("flare_nested_global_positions", first.data_ptr(), int(first.numel()), levels,
                     ctypes.cast(ptrs, ctypes.c_void_p), ctypes.cast(lengths, ctypes.c_void_p),
                     origin.data_ptr(), int(origin.numel()), ctypes.cast(dims, ctypes.c_void_p), out.data_ptr(),
                     int(s.cuda_stream))
    result = out[: int(first.numel())]
    s.synchronize()
    if result.numel() and bool((result < 0).any()):
        raise ValueError(
            f"[InputSPMD._sparse_unique:{group_name}] local row index exceeds origin length "
            f"{int(origin.numel())} or a nested index exceeds its dense width."
        )
    return result.cpu().numpy() if host_result else result
