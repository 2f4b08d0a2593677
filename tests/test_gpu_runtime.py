"""Streams and the zero fill of the C ABI (for hosts without a HIP binding of their own)."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("offset,length", [(0, 1), (1, 3), (3, 16), (16, 4096), (5, 4133), (0, 1 << 20)])
def test_zero_bytes_clears_exactly_its_range(gpu_device, no_device_errors, offset, length):
    from flare_amd import _native

    lib = _native.library()
    stream = ctypes.c_void_p()
    _native.check(lib.flare_stream_create(ctypes.byref(stream)))
    assert stream.value
    rng = np.random.default_rng(offset + length)
    host = rng.integers(1, 256, size=offset + length + 64, dtype=np.uint8)
    buf = torch.from_numpy(host.copy()).to(gpu_device)
    torch.cuda.synchronize()
    _native.check(lib.flare_zero_bytes(ctypes.c_void_p(buf.data_ptr() + offset), length, stream))
    _native.check(lib.flare_stream_synchronize(stream))
    got = buf.cpu().numpy()
    expected = host.copy()
    expected[offset:offset + length] = 0
    np.testing.assert_array_equal(got, expected)
    _native.check(lib.flare_stream_destroy(stream))
    no_device_errors()


@pytest.mark.parametrize("row_bytes,n,offset", [(256, 4099, 0), (12, 777, 4), (2, 1 << 16, 2), (512, 1, 0)])
@pytest.mark.parametrize("indexed", ["none", "src", "dst"])
def test_copy_rows_matches_indexing(gpu_device, no_device_errors, row_bytes, n, offset, indexed):
    """flare_copy_rows bit for bit against torch indexing: the contiguous path (no
    index), a gathered source and a scattered destination, with the unit width
    (16 / 8 / 4 / 2 bytes) set by the row size and the buffers' alignment."""
    from flare_amd import _native

    rows = n + 5
    rng = np.random.default_rng(row_bytes * 7 + n)
    src_all = torch.from_numpy(rng.integers(0, 256, size=rows * row_bytes + offset, dtype=np.uint8)).to(gpu_device)
    dst_all = torch.from_numpy(rng.integers(0, 256, size=rows * row_bytes + offset, dtype=np.uint8)).to(gpu_device)
    src = src_all[offset:].view(rows, row_bytes)
    dst = dst_all[offset:].view(rows, row_bytes)
    expected = dst.clone()
    src_index = dst_index = None
    if indexed == "src":
        src_index = torch.from_numpy(rng.integers(0, rows, size=n).astype(np.int32)).to(gpu_device)
        expected[:n] = src[src_index.long()]
    elif indexed == "dst":
        dst_index = torch.from_numpy(rng.permutation(rows)[:n].astype(np.int32)).to(gpu_device)
        expected[dst_index.long()] = src[:n]
    else:
        expected[:n] = src[:n]
    torch.cuda.synchronize()
    _native.call("flare_copy_rows", src.data_ptr(), rows, dst.data_ptr(), rows, row_bytes,
                 None if src_index is None else src_index.data_ptr(),
                 None if dst_index is None else dst_index.data_ptr(), n,
                 int(torch.cuda.current_stream(gpu_device).cuda_stream))
    torch.cuda.synchronize()
    assert torch.equal(dst, expected)
    no_device_errors()
