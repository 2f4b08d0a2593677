"""Checkpoint page images of the stores: export, import, assign.

The reference's store hands its checkpoint code pages of keys / values / optimizer states /
steps (tests/runtime/test_sparse_storage_limits.py:62-119, tools/validation/audit_sparse_checkpoint.py:33-70).
Known answer from the reference: zero-init Adam(lr=0.1) with gradient 1 is -0.1 after one step;
saved, restored and stepped again it is -0.2, with per-key step 1 in the saved pages.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _audit(store, pages, bound):
    """The checks of audit_sparse_checkpoint.summarize_store, restated."""
    seen = {}
    for page in pages:
        dim = page["embedding_dim"]
        keys = np.asarray(page["keys"], dtype=np.uint64).view(np.int64)
        steps = np.asarray(page["steps"], dtype=np.uint32)
        assert keys.ndim == 1 and steps.shape == keys.shape
        if not keys.size:
            continue
        values = np.asarray(page["values"]).reshape(keys.size, dim)
        opt = np.asarray(page["optimizer_states"], dtype=np.float32).reshape(keys.size, -1)
        assert (steps <= bound).all()
        for i, k in enumerate(keys.tolist()):
            assert (dim, k) not in seen
            seen[(dim, k)] = (values[i], opt[i], int(steps[i]))
    assert len(seen) == store.total_size()
    return seen


@pytest.mark.parametrize("dynamic", [False, True])
def test_adam_known_answer_through_export_and_import(gpu_device, no_device_errors, dynamic):
    from flare_amd.store import Adam, DynamicEmbeddingStore, EmbeddingStore, Zeros

    cls = DynamicEmbeddingStore if dynamic else EmbeddingStore
    kw = dict(dims=[256], value_dtype="float32", optimizer=Adam(lr=0.1), initializer=Zeros())
    store = cls(64, **kw)
    selected = np.arange(10, dtype=np.int64) * (-7 if dynamic else 1)
    store.lookup_or_insert(selected, 256)
    store.accumulate_gradients(selected, np.ones((10, 256), np.float32))
    store.optimizer_step(1)
    if dynamic:
        store.lookup_or_insert(np.arange(1000, 1040, dtype=np.int64), 256)
    pages = store.export_page_images(page_keys=17)
    seen = _audit(store, pages, bound=1)
    for k in selected.tolist():
        value, opt, step = seen[(256, k)]
        np.testing.assert_allclose(value, -0.1, rtol=1e-5, atol=1e-6)
        assert step == 1 and opt.shape == (512,) and np.isfinite(opt).all() and np.any(opt != 0)
    restored = cls(64, **kw)
    restored.import_page_images(pages)
    assert restored.total_size() == store.total_size()
    restored.accumulate_gradients(selected, np.ones((10, 256), np.float32))
    restored.optimizer_step(1)
    values, _ = restored.lookup(selected, 256)
    restored.synchronize()
    np.testing.assert_allclose(values.cpu().numpy(), -0.2, rtol=1e-5, atol=1e-6)
    no_device_errors()


@pytest.mark.parametrize("opt_name,width", [("rowwise_adagrad", 1), ("sgd", 0), ("adam", 32)])
def test_dynamic_pages_match_lookups_and_restore_exactly(gpu_device, no_device_errors, opt_name, width):
    from flare_amd.store import Adam, DynamicEmbeddingStore, RowWiseAdagrad, Sgd

    def make():
        opt = {"rowwise_adagrad": RowWiseAdagrad(lr=0.05), "sgd": Sgd(lr=0.05), "adam": Adam(lr=0.05)}[opt_name]
        return DynamicEmbeddingStore(5000, [16], value_dtype="bfloat16", optimizer=opt, seed=12)

    rng = np.random.default_rng(6)
    pool = rng.integers(-(2 ** 62), 2 ** 62, 3000, dtype=np.int64)
    store = make()
    for _ in range(2):
        keys = np.unique(rng.choice(pool, 1500))
        store.lookup_or_insert(keys, 16)
        store.accumulate_gradients(keys, rng.standard_normal((keys.size, 16), dtype=np.float32))
        store.optimizer_step(1)
    pages = store.export_page_images(page_keys=1000)
    seen = _audit(store, pages, bound=2)
    keys = np.asarray([k for _, k in seen], np.int64)
    values, _ = store.lookup(keys, 16)
    store.synchronize()
    got = np.stack([seen[(16, k)][0] for k in keys.tolist()])
    np.testing.assert_array_equal(got, values.to(torch.float32).cpu().numpy())
    assert all(seen[(16, k)][1].shape == (width,) for k in keys.tolist())
    restored = make()
    restored.import_page_images(pages)
    for s in (store, restored):  # one more identical step on both
        s.accumulate_gradients(keys[:700], np.full((700, 16), 0.25, np.float32))
        s.optimizer_step(1)
    a, _ = store.lookup(keys, 16)
    b, _ = restored.lookup(keys, 16)
    store.synchronize()
    restored.synchronize()
    np.testing.assert_array_equal(a.to(torch.float32).cpu().numpy(), b.to(torch.float32).cpu().numpy())
    no_device_errors()


def test_assign_sets_rows_and_non_finite_state_is_visible(gpu_device, no_device_errors):
    from flare_amd.store import Adam, DynamicEmbeddingStore, Zeros

    store = DynamicEmbeddingStore(16, [2], value_dtype="float32", optimizer=Adam(lr=0.1), initializer=Zeros())
    store.assign(np.asarray([3], np.int64), np.asarray([[np.nan, 1.0]], np.float32))
    values, _ = store.lookup(np.asarray([3], np.int64), 2)
    store.synchronize()
    v = values.cpu().numpy()
    assert np.isnan(v[0, 0]) and v[0, 1] == 1.0
    pages = store.export_page_images()
    assert sum(np.asarray(p["keys"]).size for p in pages) == 1
    assert np.isnan(np.asarray(pages[0]["values"])[0])
    assert store.optimizer_enabled() and store.table_dims() == [2] and store.num_slots() == 1
    no_device_errors()


def test_exported_pages_own_their_host_memory(gpu_device, no_device_errors):
    """Page arrays stay valid and unchanged after later exports and after the store is gone."""
    import gc

    from flare_amd.store import DynamicEmbeddingStore, RowWiseAdagrad

    store = DynamicEmbeddingStore(4096, [8, 24], value_dtype="float32", optimizer=RowWiseAdagrad(lr=0.1), seed=3)
    rng = np.random.default_rng(9)
    keys = np.unique(rng.integers(0, 2 ** 40, 3000, dtype=np.int64))
    for dim in (8, 24):
        store.lookup_or_insert(keys, dim)
    first = store.export_page_images(page_keys=700)
    copies = [{k: (np.array(v, copy=True) if isinstance(v, np.ndarray) else v) for k, v in p.items()} for p in first]
    store.assign(keys, np.full((keys.size, 8), 2.5, np.float32))
    second = store.export_page_images(page_keys=700)
    del store
    gc.collect()
    torch.cuda.empty_cache()
    assert sorted(int(p["embedding_dim"]) for p in first) == sorted(int(p["embedding_dim"]) for p in second)
    for page, copy in zip(first, copies):
        for name in ("keys", "values", "optimizer_states", "steps"):
            np.testing.assert_array_equal(page[name], copy[name])
    assert any(np.all(np.asarray(p["values"]) == 2.5) for p in second if int(p["embedding_dim"]) == 8)
    no_device_errors()
