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
