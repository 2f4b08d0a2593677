"""The oracle's nested global positions against the reference's vector and a dense layout."""

from __future__ import annotations

import numpy as np

from oracle import sparse_oracle as O


def test_reference_vector():
    # tests/runtime/test_sparse_input_resources.py:77-105: flat [1,2,1,3], splits [0,2,4],
    # origins [0,1], global_shape (2,2): first occurrences 0,1,3 -> origins [0,1,3]
    out = O.nested_global_positions([np.asarray([0, 2, 4])], np.asarray([0, 1, 3]), [2], np.asarray([0, 1]))
    assert out.tolist() == [0, 1, 3]


def _random_nested(rng, rows, levels, widths):
    splits = []
    count = rows
    for k in range(levels):
        lengths = rng.integers(0, widths[k] + 1, size=count)
        sp = np.zeros(count + 1, np.int64)
        sp[1:] = np.cumsum(lengths)
        splits.append(sp)
        count = int(sp[-1])
    return splits, count


def _dense_positions(splits, widths, origin):
    """Walk every path from the rows down and record each flat value's row-major offset."""
    levels = len(splits)
    strides = [1] * (levels + 1)
    for k in range(levels - 1, -1, -1):
        strides[k] = strides[k + 1] * widths[k]
    total = int(splits[-1][-1])
    out = np.full(total, -1, np.int64)

    def walk(k, entry, base):
        sp = splits[k]
        for j, child in enumerate(range(int(sp[entry]), int(sp[entry + 1]))):
            at = base + j * strides[k + 1]
            if k + 1 == levels:
                out[child] = at
            else:
                walk(k + 1, child, at)

    for r in range(len(origin)):
        walk(0, r, int(origin[r]) * strides[0])
    return out


def test_brute_force_one_to_three_levels():
    rng = np.random.default_rng(2)
    for levels in (1, 2, 3):
        widths = [int(w) for w in rng.integers(1, 6, size=levels)]
        rows = 40
        splits, total = _random_nested(rng, rows, levels, widths)
        origin = rng.permutation(200)[:rows]
        dense = _dense_positions(splits, widths, origin)
        first = np.arange(total)
        np.testing.assert_array_equal(O.nested_global_positions(splits, first, widths, origin), dense)


def test_paths_outside_the_dense_shape():
    splits = [np.asarray([0, 3, 4])]
    assert O.nested_global_positions(splits, np.asarray([0, 2, 3, 9]), [2], np.asarray([5, 6])).tolist() == \
        [10, -1, 12, -1]
    # a row past the origins
    assert O.nested_global_positions(splits, np.asarray([3]), [3], np.asarray([5])).tolist() == [-1]
