"""The oracle's key -> row map (dynamic store) pinned by closed forms and invariants.

The reference's store is external (sparse_embedding, not vendored): its key index and
initializer stream cannot be imported here.  What is pinned:
* the mixing function by the published SplitMix64 outputs for seed 1234567;
* row assignment by hand-written first-occurrence sequences and a capacity limit;
* initial values by their range, moments, determinism and independence from the batch.
"""

from __future__ import annotations

import numpy as np

from oracle import sparse_oracle as O


def test_splitmix64_published_outputs():
    # SplitMix64 (Steele, Lea, Flood 2014; Vigna's reference code): state += golden, output mix(state)
    state = np.uint64(1234567)
    outputs = []
    with np.errstate(over="ignore"):
        for _ in range(5):
            state = state + np.uint64(0x9E3779B97F4A7C15)
            outputs.append(int(O.splitmix64_mix(np.asarray([state]))[0]))
    assert outputs == [6457827717110365317, 3203168211198807973, 9817491932198370423,
                       4593380528125082431, 16408922859458223821]


def test_rows_follow_first_occurrence_across_calls():
    m = O.KeyMap(100)
    rows, fresh = m.lookup_or_insert([5, -3, 5, 2 ** 62, -3, 7])
    assert rows.tolist() == [0, 1, 0, 2, 1, 3]
    assert fresh.all()
    rows, fresh = m.lookup_or_insert([7, 8, 5, 8, -(2 ** 63) + 1])
    assert rows.tolist() == [3, 4, 0, 4, 5]
    assert fresh.tolist() == [False, True, False, True, True]
    rows, fresh = m.lookup_or_insert([9, 5], insert=False)
    assert rows.tolist() == [-1, 0] and fresh.tolist() == [False, False]


def test_int64_min_is_not_storable():
    m = O.KeyMap(10)
    rows, _ = m.lookup_or_insert([-(2 ** 63), 1])
    assert rows.tolist() == [-1, 0]


def test_row_capacity_then_later_call():
    m = O.KeyMap(3)
    rows, _ = m.lookup_or_insert([10, 11, 10, 12, 13, 14])
    assert rows.tolist() == [0, 1, 0, 2, -1, -1]
    m.row_capacity = 5  # reserve
    rows, fresh = m.lookup_or_insert([14, 13, 10])
    assert rows.tolist() == [3, 4, 0] and fresh.tolist() == [True, True, False]


def test_initial_values_are_uniform_and_in_range():
    keys = np.random.default_rng(3).integers(-(2 ** 62), 2 ** 62, 4000)
    v = O.keymap_initial_values(keys, 64, -0.01, 0.01, 7, "float32").astype(np.float64)
    assert v.min() >= -0.01 and v.max() < 0.01
    n = v.size
    sd = 0.02 / np.sqrt(12.0)
    assert abs(v.mean()) < 4 * sd / np.sqrt(n)
    assert abs(v.var() - sd ** 2) < 0.02 * sd ** 2
    # columns and keys are not correlated
    assert abs(np.corrcoef(v[:, 0], v[:, 1])[0, 1]) < 0.1
    assert abs(np.corrcoef(v[:-1, 0], v[1:, 0])[0, 1]) < 0.1


def test_initial_values_depend_only_on_key_and_seed():
    a = O.keymap_initial_values([42, 7, -9], 16, -1.0, 1.0, 5, "float32")
    b = O.keymap_initial_values([-9, 42], 16, -1.0, 1.0, 5, "float32")
    np.testing.assert_array_equal(a[0], b[1])
    np.testing.assert_array_equal(a[2], b[0])
    c = O.keymap_initial_values([42], 16, -1.0, 1.0, 6, "float32")
    assert not np.array_equal(a[0], c[0])
    # storage rounding is the float32 value rounded to nearest even
    h = O.keymap_initial_values([42], 16, -1.0, 1.0, 5, "float16")
    np.testing.assert_array_equal(h[0], a[0].astype(np.float16))
