"""Nested global positions on the GPU against the oracle (CSR-native ingest)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import sparse_oracle as O

pytestmark = pytest.mark.gpu


def test_reference_vector(gpu_device, no_device_errors):
    from flare_amd.ingest import unique_global_flat_positions

    out = unique_global_flat_positions([np.asarray([0, 2, 4], np.int32)], np.asarray([0, 1, 3], np.int64), [2],
                                       np.asarray([0, 1], np.int32), "group_dim_2")
    assert isinstance(out, np.ndarray) and out.dtype == np.int32 and out.tolist() == [0, 1, 3]
    no_device_errors()


@pytest.mark.parametrize("levels", [1, 2, 3, 4])
def test_random_nested_batches(gpu_device, no_device_errors, levels):
    from flare_amd.ingest import unique_global_flat_positions

    rng = np.random.default_rng(10 + levels)
    widths = [int(w) for w in rng.integers(1, 7, size=levels)]
    count = rows = 3000
    splits = []
    for k in range(levels):
        lengths = rng.integers(0, widths[k] + 1, size=count)
        lengths[::7] = 0
        sp = np.zeros(count + 1, np.int64)
        sp[1:] = np.cumsum(lengths)
        splits.append(sp)
        count = int(sp[-1])
    flat = rng.integers(0, 500, size=count)
    _, first = np.unique(flat, return_index=True)
    first = np.sort(first).astype(np.int64)
    origin = rng.permutation(20 * rows)[:rows].astype(np.int64)
    expected = O.nested_global_positions(splits, first, widths, origin)
    assert (expected >= 0).all()
    got = unique_global_flat_positions([torch.from_numpy(s).to(gpu_device) for s in splits],
                                       torch.from_numpy(first).to(gpu_device), widths,
                                       torch.from_numpy(origin).to(gpu_device))
    assert isinstance(got, torch.Tensor)
    np.testing.assert_array_equal(got.cpu().numpy(), expected)
    no_device_errors()


def test_errors_match_the_reference(gpu_device, no_device_errors):
    from flare_amd.ingest import unique_global_flat_positions

    with pytest.raises(ValueError, match="nested levels 1 != dense widths 2"):
        unique_global_flat_positions([np.asarray([0, 2])], np.asarray([0]), [2, 3], np.asarray([0]), "g")
    with pytest.raises(ValueError, match="exceeds origin length"):
        unique_global_flat_positions([np.asarray([0, 3, 4])], np.asarray([0, 2]), [2], np.asarray([5, 6]), "g")
    no_device_errors(1)


def test_empty_first_indices_and_empty_lists(gpu_device, no_device_errors):
    from flare_amd.ingest import unique_global_flat_positions

    out = unique_global_flat_positions([np.asarray([0, 0, 0], np.int64)], np.zeros(0, np.int64), [4],
                                       np.asarray([0, 1], np.int64))
    assert isinstance(out, np.ndarray) and out.dtype == np.int32 and out.size == 0
    # rows whose lists are all empty around one non-empty row; origins out of order
    splits = [np.asarray([0, 0, 0, 3, 3], np.int64), np.asarray([0, 2, 2, 5], np.int64)]
    first = np.asarray([0, 1, 2, 3, 4], np.int64)
    origin = np.asarray([9, 4, 7, 0], np.int64)
    expected = O.nested_global_positions(splits, first, [3, 4], origin)
    got = unique_global_flat_positions(splits, first, [3, 4], origin)
    np.testing.assert_array_equal(got, expected)
    assert got.tolist() == [7 * 12 + 0, 7 * 12 + 1, 7 * 12 + 2 * 4 + 0, 7 * 12 + 2 * 4 + 1, 7 * 12 + 2 * 4 + 2]
    no_device_errors()
