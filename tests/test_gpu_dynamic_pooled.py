"""The fused pooled step over arbitrary int64 keys on the GPU (DynamicEmbeddingStore).

keys -> key map rows (first-occurrence order, new rows initialised) -> pooled gather of the
rows -> dedup + deterministic segment sum + optimizer update of the dim's table, checked
against the oracle's KeyMap, keymap_initial_values, gather_pooled_csr and pooled_step over the
same rows; unique keys, inverse and first indices against the reference's first-occurrence
dedup of the keys themselves.
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


def _bags(rng, features, batch, max_len, pool):
    lengths = rng.integers(0 if max_len > 1 else 1, max_len + 1, size=features * batch)
    offsets = np.zeros(lengths.size + 1, np.int64)
    offsets[1:] = np.cumsum(lengths)
    # skewed draws from the pool: a few hot keys, many cold ones
    ranks = np.minimum(rng.zipf(1.3, size=int(offsets[-1])) - 1, pool.size - 1)
    return pool[ranks].astype(np.int64), offsets


CASES = [
    # value dtype, dim, features, batch, max bag length, pooling, optimizer
    ("bfloat16", 128, 3, 700, 1, "sum", "rowwise_adagrad"),
    ("bfloat16", 64, 2, 500, 4, "mean", "adam"),
    ("float16", 32, 4, 300, 6, "weighted", "sgd"),
    ("float32", 16, 1, 900, 3, "sum", "adam"),
]


@pytest.mark.parametrize("case", range(len(CASES)))
def test_dynamic_pooled_step_matches_oracle(gpu_device, no_device_errors, case):
    from flare_amd.store import Adam, DynamicEmbeddingStore, RowWiseAdagrad, Sgd, Uniform

    value_dtype, dim, features, batch, max_len, pooling, optimizer = CASES[case]
    rng = np.random.default_rng(100 + case)
    pool = rng.integers(-(2 ** 63) + 1, 2 ** 63 - 1, size=5000, dtype=np.int64)
    keys, offsets = _bags(rng, features, batch, max_len, pool)
    n = keys.size
    weights = rng.uniform(0, 1, n).astype(np.float32) if pooling == "weighted" else None
    opt = {"rowwise_adagrad": RowWiseAdagrad(lr=0.01, eps=1e-8), "adam": Adam(lr=0.01),
           "sgd": Sgd(lr=0.01)}[optimizer]
    capacity, lo, hi, seed = 6000, -0.05, 0.05, 11
    store = DynamicEmbeddingStore(capacity, [dim], value_dtype=value_dtype, optimizer=opt,
                                  initializer=Uniform(lo, hi), seed=seed)
    pooled = store.lookup_pooled(keys, offsets, batch, dim, pooling=pooling, per_sample_weights=weights)
    store.synchronize()
    table0 = _host(store.tables[dim].table.clone())

    # rows and initial values against the oracle's key map
    km = O.KeyMap(capacity)
    rows, _ = km.lookup_or_insert(keys)
    assert store.size(dim) == len(km.rows)
    present = np.asarray(sorted(km.rows, key=km.rows.get), np.int64)
    np.testing.assert_array_equal(table0[: present.size],
                                  O.keymap_initial_values(present, dim, lo, hi, seed, value_dtype))
    row_base = np.array([0, capacity], np.int64)
    bags = features * batch
    expected = O.gather_pooled_csr(table0, rows, offsets, row_base, bags, dim, storage=value_dtype,
                                   pooling=pooling, weights=weights)
    assert tuple(pooled.shape) == (features, batch, dim)
    np.testing.assert_array_equal(_host(pooled).reshape(bags, 1, dim), expected)

    grad = rng.normal(0, 1e-3, size=(features, batch, dim)).astype(np.float32)
    unique_keys, inverse, first = store.apply_pooled_gradients(
        keys, offsets, batch, torch.from_numpy(grad).to(gpu_device), dim, pooling=pooling,
        per_sample_weights=weights, return_dedup=True)
    store.synchronize()
    e_keys, e_inverse, e_first = O.unique_first_occurrence_hash(keys)
    np.testing.assert_array_equal(unique_keys.cpu().numpy(), e_keys)
    np.testing.assert_array_equal(inverse.cpu().numpy(), e_inverse)
    np.testing.assert_array_equal(first.cpu().numpy(), e_first)

    state = {}
    if optimizer == "rowwise_adagrad":
        state = {"acc": np.zeros(capacity, np.float32)}
    elif optimizer == "adam":
        state = {"m": np.zeros((capacity, dim), np.float32), "v": np.zeros((capacity, dim), np.float32),
                 "step": np.zeros(capacity, np.int32)}
    _, e_table, e_state, e_unique, _, _ = O.pooled_step(
        table0, state, rows, offsets, row_base, bags, dim, grad.reshape(bags, 1, dim), storage=value_dtype,
        pooling=pooling, weights=weights, optimizer=optimizer)
    np.testing.assert_array_equal(e_unique, rows[e_first])
    ulps = O.storage_ulp_distance(_host(store.tables[dim].table), e_table, value_dtype)
    assert ulps.max() <= 1, f"max ulp {ulps.max()}"
    s = store.tables[dim]
    if optimizer == "rowwise_adagrad":
        np.testing.assert_allclose(s.state0.cpu().numpy(), e_state["acc"], rtol=1e-5, atol=0)
    elif optimizer == "adam":
        np.testing.assert_allclose(s.state0.cpu().numpy(), e_state["m"], rtol=1e-5, atol=1e-12)
        np.testing.assert_allclose(s.state1.cpu().numpy(), e_state["v"], rtol=1e-5, atol=1e-15)
        np.testing.assert_array_equal(s.step.cpu().numpy(), e_state["step"])
    no_device_errors()


def test_dynamic_pooled_update_skips_keys_without_rows(gpu_device, no_device_errors):
    """Keys never inserted have no row: the update leaves them out (error bit 1) and updates the
    others exactly as if those occurrences were absent; the table gains no row."""
    from flare_amd.store import DynamicEmbeddingStore, Sgd, Uniform

    dim, batch = 8, 6
    store = DynamicEmbeddingStore(64, [dim], value_dtype="float32", optimizer=Sgd(lr=0.5),
                                  initializer=Uniform(-1.0, 1.0), seed=3)
    known = np.array([10, 20, 30], np.int64)
    store.lookup_or_insert(known, dim)
    store.synchronize()
    table0 = store.tables[dim].table.cpu().numpy().copy()
    keys = np.array([10, 99, 20, 10, 77, 30], np.int64)  # 99 and 77 have no row
    offsets = np.arange(batch + 1, dtype=np.int64)
    grad = np.arange(batch * dim, dtype=np.float32).reshape(1, batch, dim) / 64.0
    store.apply_pooled_gradients(keys, offsets, batch, torch.from_numpy(grad).to(gpu_device), dim)
    store.synchronize()
    table = store.tables[dim].table.cpu().numpy()
    g = grad[0]
    expected = table0.copy()
    expected[0] = (table0[0] - np.float32(0.5) * (g[0] + g[3])).astype(np.float32)
    expected[1] = (table0[1] - np.float32(0.5) * g[2]).astype(np.float32)
    expected[2] = (table0[2] - np.float32(0.5) * g[5]).astype(np.float32)
    np.testing.assert_array_equal(table, expected)
    assert store.size(dim) == 3
    no_device_errors(1)


def test_dynamic_pooled_update_rejects_nonfinite_gradients(gpu_device, no_device_errors):
    """validate_values on the pooled step over keys: an inf in the pooled gradient raises
    FloatingPointError and updates nothing; the same step with finite values then updates."""
    from flare_amd.store import DynamicEmbeddingStore, RowWiseAdagrad, Uniform

    dim, batch, features = 16, 50, 2
    rng = np.random.default_rng(5)
    keys = rng.integers(-(2 ** 40), 2 ** 40, size=features * batch).astype(np.int64)
    offsets = np.arange(keys.size + 1, dtype=np.int64)
    store = DynamicEmbeddingStore(400, [dim], value_dtype="bfloat16", optimizer=RowWiseAdagrad(lr=0.1),
                                  initializer=Uniform(-0.5, 0.5), seed=8)
    store.lookup_pooled(keys, offsets, batch, dim)
    store.synchronize()
    table0 = _host(store.tables[dim].table.clone())
    grad = torch.full((features, batch, dim), 1e-3, dtype=torch.bfloat16, device=gpu_device)
    grad[1, 7, 3] = float("inf")
    with pytest.raises(FloatingPointError):
        store.apply_pooled_gradients(keys, offsets, batch, grad, dim, validate_values=True)
    store.synchronize()
    np.testing.assert_array_equal(_host(store.tables[dim].table), table0)
    grad[1, 7, 3] = 1e-3
    store.apply_pooled_gradients(keys, offsets, batch, grad, dim, validate_values=True)
    store.synchronize()
    assert not np.array_equal(_host(store.tables[dim].table), table0)
    no_device_errors(8)
