"""The allocation-free dedup entry point (flare_unique_first_occurrence_noalloc) against the
allocating one (flare_unique_first_occurrence with a caller workspace), through the C ABI.

Two calls in a row, the second with a smaller input, so the second runs on scratch memory that
still holds the first call's contents; int64 and int32 keys; the size limit and the key_bound
requirement are refused before anything runs.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

_CODES = {torch.int64: 4, torch.int32: 3}  # FLARE_INT64, FLARE_INT32


def _outputs(n, dtype, device):
    return (torch.empty(n, dtype=dtype, device=device), torch.empty(n, dtype=torch.int32, device=device),
            torch.empty(n, dtype=torch.int64, device=device), torch.empty(1, dtype=torch.int64, device=device))


def _unique(keys: torch.Tensor, key_bound: int, noalloc: bool):
    from flare_amd import _native

    n = keys.numel()
    unique, inverse, first, count = _outputs(n, keys.dtype, keys.device)
    stream = int(torch.cuda.current_stream(keys.device).cuda_stream)
    if noalloc:
        _native.call("flare_unique_first_occurrence_noalloc", keys.data_ptr(), _CODES[keys.dtype], n, key_bound,
                     unique.data_ptr(), inverse.data_ptr(), first.data_ptr(), count.data_ptr(), stream)
    else:
        nbytes = _native.library().flare_unique_workspace_bytes(n, _CODES[keys.dtype])
        workspace = torch.empty(nbytes, dtype=torch.uint8, device=keys.device)
        _native.call("flare_unique_first_occurrence", keys.data_ptr(), _CODES[keys.dtype], n, key_bound,
                     unique.data_ptr(), inverse.data_ptr(), first.data_ptr(), count.data_ptr(),
                     workspace.data_ptr(), nbytes, stream)
    torch.cuda.synchronize()
    u = int(count.item())
    return unique[:u].cpu().numpy(), inverse.cpu().numpy(), first[:u].cpu().numpy(), u


@pytest.mark.parametrize("dtype", [torch.int64, torch.int32])
def test_noalloc_unique_matches_the_allocating_entry_point(gpu_device, no_device_errors, dtype):
    rng = np.random.default_rng(77)
    key_bound = 1 << 20
    for n in (1 << 20, 300_000):  # the full capacity, then a smaller call over leftover scratch
        ranks = np.minimum((rng.pareto(1.1, n) * 50).astype(np.int64), key_bound - 1)
        keys = torch.from_numpy(((ranks * 2654435761) % key_bound).astype(np.int64)).to(gpu_device).to(dtype)
        got = _unique(keys, key_bound, noalloc=True)
        ref = _unique(keys, key_bound, noalloc=False)
        assert got[3] == ref[3] and 0 < got[3] < n
        for a, b in zip(got[:3], ref[:3]):
            np.testing.assert_array_equal(a, b)
        k = keys.cpu().numpy()
        np.testing.assert_array_equal(got[0][got[1]], k)  # unique[inverse] == keys
    no_device_errors()


def test_noalloc_unique_refuses_what_it_cannot_hold(gpu_device):
    from flare_amd import _native

    with pytest.raises(ValueError, match="key_bound > 0"):
        _native.call("flare_unique_first_occurrence_noalloc", None, 4, 10, 0, None, None, None, None, None)
    with pytest.raises(ValueError, match="at most 1048576 keys"):
        _native.call("flare_unique_first_occurrence_noalloc", None, 4, (1 << 20) + (1 << 16), 1 << 20, None, None,
                     None, None, None)
