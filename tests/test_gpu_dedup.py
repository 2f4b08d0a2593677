"""GPU dedup: bit-exact first-occurrence unique / inverse / first_indices.

Cases of tests/runtime/test_sparse_input_resources.py:77-143 in the
reference, then random inputs checked against both oracle formulations.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import sparse_oracle as O

pytestmark = pytest.mark.gpu

REFERENCE_CASES = (
    np.asarray([], dtype=np.int64),
    np.asarray([7, 7, 7], dtype=np.int64),
    np.asarray([3, 1, 3, 2, 1], dtype=np.int64),
    np.asarray([-1, 0, -1, np.iinfo(np.int64).min], dtype=np.int64),
    np.asarray([2**63, 0, 2**63, 2**64 - 1], dtype=np.uint64),
    np.asarray([1, 2, 1, 3], dtype=np.int64),
)


@pytest.mark.parametrize("case", range(len(REFERENCE_CASES)))
def test_reference_cases(gpu_device, no_device_errors, case):
    from flare_amd.unique import unique_first_occurrence

    values = REFERENCE_CASES[case]
    unique, inverse, first = unique_first_occurrence(values)
    assert np.array_equal(unique[inverse], values)
    assert np.array_equal(values[first], unique)
    assert inverse.dtype == np.int32 and first.dtype == np.int64 and unique.dtype == values.dtype
    eu, ei, ef = O.unique_first_occurrence_hash(values)
    np.testing.assert_array_equal(unique, eu)
    np.testing.assert_array_equal(inverse, ei)
    np.testing.assert_array_equal(first, ef)
    no_device_errors()


def test_routing_contract_vector(gpu_device):
    from flare_amd.unique import unique_first_occurrence

    unique, inverse, first = unique_first_occurrence(np.asarray([1, 2, 1, 3], dtype=np.int64))
    assert unique.tolist() == [1, 2, 3]
    assert inverse.tolist() == [0, 1, 0, 2]
    assert first.tolist() == [0, 1, 3]


def test_rejects_non_integer_keys(gpu_device):
    from flare_amd.unique import unique_first_occurrence

    with pytest.raises(TypeError):
        unique_first_occurrence(np.asarray([1.0, 2.0]))


@pytest.mark.parametrize("dtype", [np.int32, np.uint32, np.int64, np.uint64])
@pytest.mark.parametrize("n,span,seed", [(1, 5, 0), (4095, 100, 1), (4097, 10**6, 2), (50000, 300, 3), (200000, 2**40, 4)])
def test_random_keys_bit_exact(gpu_device, no_device_errors, dtype, n, span, seed):
    from flare_amd.unique import unique_first_occurrence

    rng = np.random.default_rng(seed)
    info = np.iinfo(dtype)
    hi = min(span, int(info.max))
    values = rng.integers(0, hi, n, dtype=np.uint64).astype(dtype)
    if np.dtype(dtype).kind == "i":
        values = (values.astype(np.int64) - hi // 2).astype(dtype)
    unique, inverse, first = unique_first_occurrence(values)
    eu, ei, ef = O.unique_first_occurrence_sorted(values)
    np.testing.assert_array_equal(unique, eu)
    np.testing.assert_array_equal(inverse, ei)
    np.testing.assert_array_equal(first, ef)
    no_device_errors()


def test_device_input_and_key_bound(gpu_device, no_device_errors):
    from flare_amd.unique import unique_first_occurrence

    rng = np.random.default_rng(7)
    values = rng.integers(0, 5000, 123457).astype(np.int64)
    dev = torch.from_numpy(values).to(gpu_device)
    for bound in (0, 5000):
        unique, inverse, first = unique_first_occurrence(dev, key_bound=bound)
        eu, ei, ef = O.unique_first_occurrence_sorted(values)
        np.testing.assert_array_equal(unique.cpu().numpy(), eu)
        np.testing.assert_array_equal(inverse.cpu().numpy(), ei)
        np.testing.assert_array_equal(first.cpu().numpy(), ef)
    no_device_errors()


@pytest.mark.parametrize("bits", [9, 10, 16, 17, 18, 19, 20, 24, 25, 26, 27, 28, 30, 32, 36])
def test_every_radix_plan(gpu_device, no_device_errors, bits):
    """Key widths that select each digit width (8, 9, 10 bits) and pass count, 32- and 64-bit keys."""
    from flare_amd.unique import unique_first_occurrence

    rng = np.random.default_rng(bits)
    n = 70000
    values = rng.integers(0, 1 << bits, n, dtype=np.uint64).astype(np.int64)
    values[rng.random(n) < 0.3] = 0  # a hot key at the bottom of the range
    values[0], values[1] = 0, (1 << bits) - 1  # span exactly `bits` bits
    unique, inverse, first = unique_first_occurrence(values)
    eu, ei, ef = O.unique_first_occurrence_sorted(values)
    np.testing.assert_array_equal(unique, eu)
    np.testing.assert_array_equal(inverse, ei)
    np.testing.assert_array_equal(first, ef)
    no_device_errors()


@pytest.mark.parametrize("dtype,span", [(np.int32, 1 << 22), (np.int64, 1 << 40)])
def test_more_tiles_than_the_fused_prefix_covers(gpu_device, no_device_errors, dtype, span):
    """2049 tiles of 4096 occurrences and a ragged tail: the runs and ranks take their tile
    prefixes from separate scan launches (up to 2048 tiles the kernels add them up
    themselves).  Expected values restate the reference's GPU branch: np.unique with first
    indices and inverse, then ranks in first-occurrence order."""
    from flare_amd.unique import unique_first_occurrence

    rng = np.random.default_rng(77)
    n = 2049 * 4096 + 123
    values = rng.integers(0, span, size=n).astype(dtype)
    values[rng.random(n) < 0.3] = values[0]  # one heavy key
    u_sorted, first_idx, inv_sorted = np.unique(values, return_index=True, return_inverse=True)
    order = np.argsort(first_idx, kind="stable")
    rank_of_sorted = np.empty_like(order)
    rank_of_sorted[order] = np.arange(order.size)
    unique, inverse, first = unique_first_occurrence(torch.from_numpy(values).to(gpu_device))
    np.testing.assert_array_equal(unique.cpu().numpy(), u_sorted[order])
    np.testing.assert_array_equal(first.cpu().numpy(), first_idx[order])
    np.testing.assert_array_equal(inverse.cpu().numpy(), rank_of_sorted[inv_sorted.reshape(-1)])
    no_device_errors()


@pytest.mark.parametrize("bad", [-1, 50, 1 << 40])
def test_key_bound_violation_sets_the_error_bit(gpu_device, no_device_errors, bad):
    """key_bound promises 0 <= key < key_bound; a key outside it is reported (device error bit 1)
    instead of silently splitting its run."""
    from flare_amd.unique import unique_first_occurrence

    keys = torch.tensor([3, 7, bad, 3, 9], dtype=torch.int64, device=gpu_device)
    unique_first_occurrence(keys, key_bound=50)
    no_device_errors(1)
    unique_first_occurrence(torch.tensor([3, 7, 49, 3], dtype=torch.int64, device=gpu_device), key_bound=50)
    no_device_errors(0)
