"""GPU store update: accumulate_gradients + optimizer_step against the oracle.

Known answers of the reference: zero-init Adam(lr=0.1) with grad 1 gives
-0.1 after one step and -0.2 after two (tests/runtime/test_sparse_storage_limits.py:41-119);
SGD(lr=1) flush of a partial window (tests/training/test_checkpointing.py:229-298).
"""

from __future__ import annotations

import asyncio

import numpy as np
import pytest
import torch

from oracle import sparse_oracle as O

pytestmark = pytest.mark.gpu


def _store(**kw):
    from flare_amd.store import EmbeddingStore

    return EmbeddingStore(**kw)


def test_adam_known_answer(gpu_device, no_device_errors):
    from flare_amd.store import Adam, Zeros

    for dim in (4, 256):
        store = _store(capacity=40000, dims=[dim], value_dtype="float32", optimizer=Adam(lr=0.1),
                       initializer=Zeros())
        selected = np.arange(10, dtype=np.int64)
        store.lookup_or_insert(selected, dim)
        store.accumulate_gradients(selected, np.ones((10, dim), dtype=np.float32))
        store.optimizer_step(1)
        values, _ = store.lookup(selected, dim)
        store.synchronize()
        np.testing.assert_allclose(values.cpu().numpy(), -0.1, rtol=1e-5, atol=1e-6)
        state = store.tables[dim]
        assert (state.step[:10].cpu().numpy() == 1).all()
        assert (state.step[10:].cpu().numpy() == 0).all()
        store.accumulate_gradients(selected, np.ones((10, dim), dtype=np.float32))
        store.optimizer_step(1)
        values, _ = store.lookup(selected, dim)
        store.synchronize()
        np.testing.assert_allclose(values.cpu().numpy(), -0.2, rtol=1e-5, atol=1e-6)
        untouched, _ = store.lookup(np.arange(10, 20), dim)
        store.synchronize()
        assert (untouched.cpu().numpy() == 0).all()
    no_device_errors()


@pytest.mark.parametrize("value_dtype", ["float16", "float32", "bfloat16"])
def test_sgd_partial_window_and_dtype(gpu_device, no_device_errors, value_dtype):
    from flare_amd.store import Sgd, Uniform

    store = _store(capacity=16, dims=[2], value_dtype=value_dtype, optimizer=Sgd(lr=1.0),
                   initializer=Uniform(0.0, 0.0))

    async def run():
        keys = np.asarray([7], dtype=np.int64)
        await store.async_accumulate_gradients(keys, np.asarray([[1.0, 2.0]], dtype=np.float32))
        await store.async_optimizer_step(1)
        values, _ = await store.async_lookup(keys, 2)
        return values

    values = asyncio.run(run())
    store.synchronize()
    assert str(values.dtype).endswith(value_dtype)
    np.testing.assert_array_equal(values.to(torch.float32).cpu().numpy(), [[-1.0, -2.0]])
    assert store.value_dtype() == value_dtype and store.optimizer_dtype() == "float32"
    no_device_errors()


@pytest.mark.parametrize("opt", ["adam", "sgd", "rowwise_adagrad"])
@pytest.mark.parametrize("value_dtype", ["float32", "bfloat16", "float16"])
def test_multi_microstep_update_matches_oracle(gpu_device, no_device_errors, opt, value_dtype):
    from flare_amd.store import Adam, RowWiseAdagrad, Sgd

    rows, dim = 3000, 64
    optimizer = {"adam": Adam(lr=0.01), "sgd": Sgd(lr=0.05), "rowwise_adagrad": RowWiseAdagrad(lr=0.01)}[opt]
    store = _store(capacity=rows, dims=[dim], value_dtype=value_dtype, optimizer=optimizer, seed=5)
    table0 = store.tables[dim].table.clone()
    rng = np.random.default_rng(11)
    micro = []
    for _ in range(3):
        keys = np.minimum(rng.zipf(1.2, 5000) - 1, rows - 1).astype(np.int64)
        grad = rng.standard_normal((keys.size, dim), dtype=np.float32) * np.float32(1e-3)
        micro.append((keys, grad))
        store.accumulate_gradients(keys, grad)
    store.optimizer_step(3)
    store.synchronize()
    # oracle: keyed sum of all micro-steps in occurrence order, / 3, then optimizer
    keys = np.concatenate([k for k, _ in micro])
    grad = np.concatenate([g for _, g in micro])
    perm, sk, starts = O.sorted_occurrences(keys)
    sums = (O.segment_sums(grad[perm], starts, perm.size) / np.float32(3)).astype(np.float32)
    rows_touched = sk[starts]
    host0 = table0.view(torch.int16).cpu().numpy().view(np.uint16) if value_dtype == "bfloat16" else table0.cpu().numpy()
    w = O.storage_to_f32(host0[rows_touched], value_dtype)
    state = store.tables[dim]
    if opt == "adam":
        w2, m2, v2, s2 = O.adam_update(w, np.zeros_like(w), np.zeros_like(w), np.zeros(w.shape[0], np.int32), sums, lr=0.01)
        np.testing.assert_allclose(state.state0.cpu().numpy()[rows_touched], m2, rtol=1e-5, atol=1e-12)
        np.testing.assert_allclose(state.state1.cpu().numpy()[rows_touched], v2, rtol=1e-5, atol=1e-15)
        assert (state.step.cpu().numpy()[rows_touched] == 1).all()
    elif opt == "sgd":
        w2 = O.sgd_update(w, sums, lr=0.05)
    else:
        w2, acc2 = O.rowwise_adagrad_update(w, np.zeros(w.shape[0], np.float32), sums, lr=0.01)
        np.testing.assert_allclose(state.state0.cpu().numpy()[rows_touched], acc2, rtol=1e-5)
    table = state.table
    got = table.view(torch.int16).cpu().numpy().view(np.uint16) if value_dtype == "bfloat16" else table.cpu().numpy()
    expected = O.f32_to_storage(w2, value_dtype)
    ulps = O.storage_ulp_distance(got[rows_touched], expected, value_dtype)
    assert ulps.max() <= 1, f"max ulp distance {ulps.max()}"
    untouched = np.setdiff1d(np.arange(rows), rows_touched)
    np.testing.assert_array_equal(got[untouched], host0[untouched])
    no_device_errors()


@pytest.mark.parametrize("dim", [16, 64, 128])
@pytest.mark.parametrize("count,repeat", [(300, 1), (700, 1), (65, 1), (4097, 1), (700, 3)])
def test_every_key_updated_once_for_any_key_count(gpu_device, no_device_errors, dim, count, repeat):
    """Key counts that split unevenly over the lane groups of a wave (single-occurrence keys
    and, with repeat 3, keys of several occurrences): every touched row equals the oracle's
    one row-wise Adagrad step, every other row is unchanged."""
    from flare_amd.store import RowWiseAdagrad

    rows = 8192
    store = _store(capacity=rows, dims=[dim], value_dtype="float32", optimizer=RowWiseAdagrad(lr=0.01), seed=3)
    table0 = store.tables[dim].table.cpu().numpy().copy()
    rng = np.random.default_rng(count * 7 + dim + repeat)
    distinct = rng.permutation(rows)[:count].astype(np.int64)
    keys = np.concatenate([distinct] * repeat)
    grad = rng.standard_normal((keys.size, dim), dtype=np.float32)
    store.accumulate_gradients(keys, grad)
    store.optimizer_step(1)
    store.synchronize()
    perm, sk, starts = O.sorted_occurrences(keys)
    sums = O.segment_sums(grad[perm], starts, perm.size)
    touched = sk[starts]
    w2, acc2 = O.rowwise_adagrad_update(table0[touched], np.zeros(touched.size, np.float32), sums, lr=0.01)
    got = store.tables[dim].table.cpu().numpy()
    ulps = O.storage_ulp_distance(got[touched], w2, "float32")
    assert ulps.max() <= 1, f"max ulp distance {ulps.max()}"
    np.testing.assert_allclose(store.tables[dim].state0.cpu().numpy()[touched], acc2, rtol=1e-5)
    untouched = np.setdiff1d(np.arange(rows), touched)
    np.testing.assert_array_equal(got[untouched], table0[untouched])
    no_device_errors()


def test_rejects_bad_normalization_and_shapes(gpu_device):
    from flare_amd.store import Adam

    store = _store(capacity=8, dims=[4], optimizer=Adam())
    with pytest.raises(ValueError):
        store.optimizer_step(0)
    with pytest.raises(ValueError):
        store.accumulate_gradients(np.arange(3), np.ones((2, 4), np.float32))
    with pytest.raises(ValueError):
        store.reserve(9, 4)
