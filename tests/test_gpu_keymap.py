"""Dynamic store on the GPU: key -> row map and store updates against the oracle's KeyMap.

Rows are bit-exact (first-occurrence order per call), initial values bit-exact against
``keymap_initial_values``, later lookups return the stored rows.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import sparse_oracle as O

pytestmark = pytest.mark.gpu


def _host(t: torch.Tensor) -> np.ndarray:
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).cpu().numpy().view(np.uint16)
    return t.cpu().numpy()


def _keys(rng, pool, n):
    return rng.choice(pool, size=n, replace=True).astype(np.int64)


@pytest.mark.parametrize("value_dtype,dim", [("bfloat16", 128), ("float16", 64), ("float32", 20), ("float32", 36)])
def test_lookup_or_insert_matches_oracle(gpu_device, no_device_errors, value_dtype, dim):
    from flare_amd.store import DynamicEmbeddingStore, Sgd, Uniform

    rng = np.random.default_rng(17)
    pool = rng.integers(-(2 ** 63) + 1, 2 ** 63 - 1, size=9000, dtype=np.int64)
    pool[:4] = [0, -1, 2 ** 63 - 1, -(2 ** 63) + 1]
    store = DynamicEmbeddingStore(20000, [dim], value_dtype=value_dtype, optimizer=Sgd(),
                                  initializer=Uniform(-0.05, 0.03), seed=99)
    oracle = O.KeyMap(20000)
    expected_rows = {}
    for call in range(3):
        keys = _keys(rng, pool[: 3000 * (call + 1)], 7000)
        values, _ = store.lookup_or_insert(keys, dim)
        rows = store.rows(keys, dim)
        store.synchronize()
        e_rows, _ = oracle.lookup_or_insert(keys)
        np.testing.assert_array_equal(rows.cpu().numpy(), e_rows)
        for k, r in zip(keys.tolist(), e_rows.tolist()):
            expected_rows[k] = r
        e_values = O.keymap_initial_values(keys, dim, -0.05, 0.03, 99, value_dtype)
        np.testing.assert_array_equal(_host(values), e_values)
    assert store.size(dim) == len(oracle.rows)
    # the table holds each key's initial row at its row
    all_keys = np.asarray(list(expected_rows), np.int64)
    table = _host(store.tables[dim].table)
    np.testing.assert_array_equal(table[[expected_rows[k] for k in all_keys.tolist()]],
                                  O.keymap_initial_values(all_keys, dim, -0.05, 0.03, 99, value_dtype))
    no_device_errors()


def test_lookup_of_absent_keys_and_contains(gpu_device, no_device_errors):
    from flare_amd.store import DynamicEmbeddingStore, Sgd

    store = DynamicEmbeddingStore(100, [8], value_dtype="float32", optimizer=Sgd(), seed=1)
    store.lookup_or_insert(np.asarray([3, 1 << 40, -5], np.int64), 8)
    values, _ = store.lookup(np.asarray([-5, 4, 1 << 40], np.int64), 8)
    rows = store.rows(np.asarray([-5, 4, 1 << 40], np.int64), 8)
    store.synchronize()
    assert rows.cpu().numpy().tolist() == [2, -1, 1]
    v = values.cpu().numpy()
    assert (v[1] == 0).all() and not (v[0] == 0).all()
    assert store.contains(np.asarray([3, 4, -5], np.int64), 8).tolist() == [True, False, True]
    assert store.size() == 3
    no_device_errors()


def test_full_table_leaves_keys_without_rows_until_reserve(gpu_device, no_device_errors):
    from flare_amd.store import DynamicEmbeddingStore, Sgd

    store = DynamicEmbeddingStore(40, [16], value_dtype="bfloat16", optimizer=Sgd(), seed=2)
    oracle = O.KeyMap(40)
    keys = np.arange(1000, 1100, dtype=np.int64)[::-1].copy()
    rows = store.rows(keys, 16, insert=True)
    store.synchronize()
    e_rows, _ = oracle.lookup_or_insert(keys)
    np.testing.assert_array_equal(rows.cpu().numpy(), e_rows)
    no_device_errors(4)
    assert store.size(16) == 40
    store.reserve(1000, 16)  # grows the table and rehashes the map into more slots
    oracle.row_capacity = 1000
    more = np.concatenate([keys[30:70], np.arange(5000, 5100, dtype=np.int64)])
    values, _ = store.lookup_or_insert(more, 16)
    rows = store.rows(more, 16)
    store.synchronize()
    e_rows, _ = oracle.lookup_or_insert(more)
    np.testing.assert_array_equal(rows.cpu().numpy(), e_rows)
    np.testing.assert_array_equal(_host(values), O.keymap_initial_values(more, 16, -0.01, 0.01, 2, "bfloat16"))
    assert store.tables[16].rows == 1000 and store.size(16) == len(oracle.rows)
    no_device_errors()


@pytest.mark.parametrize("opt", ["adam", "rowwise_adagrad"])
def test_dynamic_store_update_matches_oracle(gpu_device, no_device_errors, opt):
    """lookup_or_insert -> accumulate_gradients x2 -> optimizer_step(2) on arbitrary keys."""
    from flare_amd.store import Adam, DynamicEmbeddingStore, RowWiseAdagrad

    dim = 64
    optimizer = Adam(lr=0.01) if opt == "adam" else RowWiseAdagrad(lr=0.01)
    store = DynamicEmbeddingStore(5000, [dim], value_dtype="float32", optimizer=optimizer, seed=4)
    oracle = O.KeyMap(5000)
    rng = np.random.default_rng(8)
    pool = rng.integers(-(2 ** 60), 2 ** 60, size=3000, dtype=np.int64)
    micro = []
    for _ in range(2):
        keys = np.unique(_keys(rng, pool, 2500))  # the worker's unique ids of one micro-step
        rng.shuffle(keys)
        store.lookup_or_insert(keys, dim)
        oracle.lookup_or_insert(keys)
        grad = rng.standard_normal((keys.size, dim), dtype=np.float32) * np.float32(1e-3)
        store.accumulate_gradients(keys, grad)
        micro.append((keys, grad))
    store.optimizer_step(2)
    store.synchronize()
    keys = np.concatenate([k for k, _ in micro])
    grad = np.concatenate([g for _, g in micro])
    rows = np.asarray([oracle.rows[k] for k in keys.tolist()], np.int64)
    perm, srows, starts = O.sorted_occurrences(rows)
    sums = (O.segment_sums(grad[perm], starts, perm.size) / np.float32(2)).astype(np.float32)
    touched = srows[starts]
    inv = {r: k for k, r in oracle.rows.items()}
    w = O.keymap_initial_values(np.asarray([inv[r] for r in touched.tolist()], np.int64), dim, -0.01, 0.01, 4,
                                "float32")
    state = store.tables[dim]
    if opt == "adam":
        w2, m2, v2, _ = O.adam_update(w, np.zeros_like(w), np.zeros_like(w), np.zeros(w.shape[0], np.int32), sums,
                                      lr=0.01)
        np.testing.assert_allclose(state.state0.cpu().numpy()[touched], m2, rtol=1e-5, atol=1e-12)
    else:
        w2, acc2 = O.rowwise_adagrad_update(w, np.zeros(w.shape[0], np.float32), sums, lr=0.01)
        np.testing.assert_allclose(state.state0.cpu().numpy()[touched], acc2, rtol=1e-5)
    got = state.table.cpu().numpy()[touched]
    assert O.storage_ulp_distance(got, w2, "float32").max() <= 1
    no_device_errors()


def test_gradient_for_a_key_without_row_is_reported(gpu_device, no_device_errors):
    from flare_amd.store import DynamicEmbeddingStore, Sgd

    store = DynamicEmbeddingStore(10, [4], value_dtype="float32", optimizer=Sgd(lr=1.0), seed=0)
    store.lookup_or_insert(np.asarray([11], np.int64), 4)
    before, _ = store.lookup(np.asarray([11], np.int64), 4)
    store.accumulate_gradients(np.asarray([11, 12], np.int64), np.ones((2, 4), np.float32))
    store.optimizer_step(1)
    after, _ = store.lookup(np.asarray([11, 12], np.int64), 4)
    store.synchronize()
    np.testing.assert_allclose(after.cpu().numpy()[0], before.cpu().numpy()[0] - 1.0, rtol=1e-6)
    assert (after.cpu().numpy()[1] == 0).all()
    no_device_errors(1)


def test_int64_min_is_not_storable(gpu_device, no_device_errors):
    """INT64_MIN marks empty slots: it gets no row (row -1, zero values) and sets error bit 1,
    while the other keys of the call are inserted in first-occurrence order as usual."""
    from flare_amd.store import DynamicEmbeddingStore, Sgd

    lo = np.iinfo(np.int64).min
    keys = np.asarray([7, lo, -7, lo, 7, 2 ** 62], np.int64)
    store = DynamicEmbeddingStore(64, [8], value_dtype="float32", optimizer=Sgd(), seed=5)
    oracle = O.KeyMap(64)
    values, _ = store.lookup_or_insert(keys, 8)
    rows = store.rows(keys, 8)
    store.synchronize()
    e_rows, _ = oracle.lookup_or_insert(keys)
    np.testing.assert_array_equal(rows.cpu().numpy(), e_rows)
    assert e_rows.tolist() == [0, -1, 1, -1, 0, 2]
    v = values.cpu().numpy()
    assert (v[[1, 3]] == 0).all()
    np.testing.assert_array_equal(v[[0, 2, 5]], O.keymap_initial_values(keys[[0, 2, 5]], 8, -0.01, 0.01, 5, "float32"))
    assert store.size(8) == 3 and store.contains(np.asarray([lo], np.int64), 8).tolist() == [False]
    no_device_errors(1)
