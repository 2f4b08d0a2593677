"""The reference's unchanged callers, replayed against the HIP operator and store on the GPU.

- ``materialize_recsys_sparse_inputs`` (``recipes/recsys/ranking/schema/materialization.py:36-79``)
  and ``scatter_sparse_grads`` (``recipes/recsys/ranking/workers/train_worker.py:478-530``):
  DLPack capsules in, ``array`` / ``inverse`` / ``gather_pooled`` / ``local_array`` /
  ``scatter_pooled`` under ``execution_context``, the keyed sum cast to the transport dtype
  with ``np.dtype(grad.dtype)`` / ``grad.astype(...)``, one ``stream.synchronize()``.
- ``DynamicSparseEmbeddingSPMD`` (``src/flare/runtime/fluxway/workers/dynamic_embedding.py:250-302,
  362-438,481-549``): ``se.EmbeddingStore(embedding_config=..., initializer_config=...,
  optimizer_config=..., score_policy="lfu")``, ``reserve``, ``async_lookup_or_insert`` with a
  capsule, ``async_accumulate_gradients(keys, capsule)`` per micro-step and
  ``async_optimizer_step(normalization_steps)`` at the window boundary.
- The reference's own store tests, restated: value / gradient dtype independence and the
  flushed partial window (``tests/training/test_checkpointing.py:229-298``), the Adam known
  answer (``tests/runtime/test_sparse_storage_limits.py:41-119``).
- Inputs produced on another stream behind a delaying kernel are read only once ready, and
  results are ordered before the caller's stream, with no ``synchronize()``.
"""

from __future__ import annotations

import asyncio
import importlib
import sys

import numpy as np
import pytest
import torch

from flare_amd.array import DeviceArray
from flare_amd.precision import prepare_sparse_native_gradient, require_sparse_tensor_dtype
from oracle import sparse_oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture()
def se():
    saved = {k: sys.modules.get(k) for k in ("sparse_embedding", "sparse_embedding.checkpoint")}
    import flare_amd.sparse_embedding as facade

    facade.install()
    yield importlib.import_module("sparse_embedding")
    for k, v in saved.items():
        if v is None:
            sys.modules.pop(k, None)
        else:
            sys.modules[k] = v


def _capsule(t: torch.Tensor):
    """A legacy DLPack capsule, as fluxway's prepare_dlpack_input hands buffers over."""
    return torch.utils.dlpack.to_dlpack(t)


def _bits(x) -> np.ndarray:
    t = x.tensor if isinstance(x, DeviceArray) else x
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).cpu().numpy().view(np.uint16)
    return t.cpu().numpy()


@pytest.mark.parametrize("transport", ["float32", "bfloat16"])
def test_train_worker_sequence(gpu_device, no_device_errors, transport):
    from flare_amd.factory import create_sparse_embedding_operator

    rng = np.random.default_rng(17)
    batch, features, max_el, dim, rows = 48, 3, 4, 16, 50
    sparse_op = create_sparse_embedding_operator("hip", value_dtype="float16", gradient_dtype="float32",
                                                 empty_cache=False)
    sparse_op.prewarm()
    # ---- materialize_recsys_sparse_inputs (materialization.py:41-79)
    emb_host = rng.uniform(-1, 1, size=(rows, dim)).astype(np.float16)
    emb_dev = torch.from_numpy(emb_host).to(gpu_device)
    valid_count_device = sparse_op.array(_capsule(torch.tensor([batch], dtype=torch.int64, device=gpu_device)))
    assert int(valid_count_device[0]) == batch
    embedding_array = sparse_op.array(_capsule(emb_dev))
    assert embedding_array.ndim == 2
    lengths = rng.integers(0, max_el + 2, size=batch * features)
    splits0 = np.arange(0, batch * features + 1, features, dtype=np.int64)
    splits1 = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int64)
    flat = rng.integers(0, rows, size=int(splits1[-1])).astype(np.int32)
    padded_inverse = O.materialize_padded_inverse(flat, [splits0, splits1], pad_index=int(embedding_array.shape[0]),
                                                  batch_size=batch, target_widths=(features, max_el))
    assert padded_inverse.dtype == sparse_op.inverse_host_dtype
    admission_inverse = sparse_op.inverse(padded_inverse)
    sparse_input = sparse_op.gather_pooled(embedding_array, admission_inverse, batch,
                                           int(embedding_array.shape[-1]), (features, max_el),
                                           int(embedding_array.shape[0]))
    sparse_input = require_sparse_tensor_dtype(sparse_input, sparse_op.value_dtype, boundary="model_gather:g")
    exported = torch.from_dlpack(sparse_input)  # what the JAX binding imports, zero-copy
    assert exported.data_ptr() == sparse_input.data_ptr()
    sparse_op.stream.synchronize()
    np.testing.assert_array_equal(exported.cpu().numpy(),
                                  O.gather_pooled(emb_host, padded_inverse, batch, dim, (features, max_el), rows,
                                                  storage="float16"))
    # ---- scatter_sparse_grads (train_worker.py:478-530)
    grad_f32 = rng.normal(0, 1, size=(batch, features, dim)).astype(np.float32)
    model_grad = torch.from_numpy(grad_f32).to(gpu_device).to(getattr(torch, transport))
    with sparse_op.execution_context() as stream:
        gradient_array = prepare_sparse_native_gradient(
            sparse_op.local_array(_capsule(model_grad)), transport_dtype=transport, native_dtype="float32")
        embedding_ref = sparse_op.local_array(_capsule(emb_dev))
        emb_dim = int(embedding_ref.shape[-1])
        grad = sparse_op.scatter_pooled(int(embedding_ref.shape[0]), emb_dim, sparse_op.inverse(padded_inverse),
                                        int(embedding_ref.shape[0]), gradient_array, (features, max_el))
        grad = require_sparse_tensor_dtype(grad, sparse_op.gradient_dtype, boundary="model_gradient_scatter:g")
        if np.dtype(grad.dtype).name != transport:
            grad = grad.astype(transport)
        grad = require_sparse_tensor_dtype(grad, transport, boundary="model_gradient_transport:g")
        if stream is not None:
            stream.synchronize()
    widened = model_grad.to(torch.float32).cpu().numpy()
    expected = O.scatter_pooled(rows, dim, padded_inverse, rows, widened, (features, max_el))
    if transport == "bfloat16":
        np.testing.assert_array_equal(_bits(grad), O.f32_to_bf16_bits(expected))
    else:
        np.testing.assert_array_equal(_bits(grad), expected)
    no_device_errors()


def _worker_store(se, value_dtype, optimizer_config, dims=(8,), low=-0.01, high=0.01, gradient_dtype="float32"):
    """The worker's construction (dynamic_embedding.py:250-276), with its required-method check."""
    embedding_config = se.EmbeddingConfig(
        dims=list(dims), thread_budget=2, value_dtype=value_dtype, gradient_dtype=gradient_dtype,
        optimizer_dtype="float32", key_dtype="int64",
        storage=se.AutoStorage(memory_limit_bytes=None, spill_directory=None, max_spill_bytes=None),
        enable_optimizer=True,
    )
    store = se.EmbeddingStore(embedding_config=embedding_config,
                              initializer_config=se.Uniform(min_val=low, max_val=high),
                              optimizer_config=optimizer_config, score_policy="lfu")
    for name in ("lookup_or_insert", "accumulate_gradients", "optimizer_step"):
        assert hasattr(store, name), name
    return store


@pytest.mark.parametrize("value_dtype", ["float32", "float16", "bfloat16"])
def test_dynamic_embedding_sequence(gpu_device, no_device_errors, se, value_dtype):
    rng = np.random.default_rng(23)
    dim, steps = 8, 2
    store = _worker_store(se, value_dtype, se.Sgd(lr=0.5, weight_decay=0.0, dynamic_lr_policy=se.ConstantLrPolicy()),
                          dims=(dim,))
    store.reserve(300, dim)
    keys = rng.integers(-(2 ** 62), 2 ** 62, size=64).astype(np.int64)
    keys = np.concatenate([keys, keys[:20]])  # duplicates within the step's keys
    # lookup (dynamic_embedding.py:385-420)
    embed_capsule, _ = asyncio.run(store.async_lookup_or_insert(keys.__dlpack__(), dim))
    embed_tensor = torch.from_dlpack(embed_capsule).reshape((-1, dim))
    assert require_sparse_tensor_dtype(embed_capsule, value_dtype, boundary="sparse_lookup") is embed_capsule
    initial = O.keymap_initial_values(keys, dim, -0.01, 0.01, 0, value_dtype)
    np.testing.assert_array_equal(_bits(embed_tensor), initial)
    # update: micro-steps then the boundary (dynamic_embedding.py:505-549)
    grads = [rng.normal(0, 1, size=(keys.size, dim)).astype(np.float32) for _ in range(steps)]
    for g in grads:
        native = prepare_sparse_native_gradient(g, transport_dtype="float32", native_dtype="float32")
        asyncio.run(store.async_accumulate_gradients(keys, np.ascontiguousarray(native).__dlpack__()))
    asyncio.run(store.async_optimizer_step(steps))
    values_capsule, _ = asyncio.run(store.async_lookup(keys.__dlpack__(), dim))
    got = _bits(values_capsule)
    uniq, inv = np.unique(keys, return_inverse=True)
    total = np.zeros((uniq.size, dim), np.float64)
    for g in grads:
        np.add.at(total, inv, g.astype(np.float64))
    w0 = O.storage_to_f32(initial, value_dtype)
    expected = (w0 - 0.5 * (total[inv] / steps)).astype(np.float32)
    if value_dtype == "float32":  # fp32 sums in another order than the float64 reference
        np.testing.assert_allclose(got, expected, rtol=2e-6, atol=1e-7)
    else:
        ulps = O.storage_ulp_distance(got, O.f32_to_storage(expected, value_dtype), value_dtype)
        assert ulps.max() <= 1, f"max ulp {ulps.max()}"
    no_device_errors()


def test_value_dtype_independent_of_gradient_dtype(gpu_device, no_device_errors, se):
    """tests/training/test_checkpointing.py:255-298, restated on the HIP store."""
    keys = np.asarray([7], dtype=np.int64)
    for value_dtype, gradient_dtype in (("float16", "float16"), ("float16", "float32"),
                                        ("float32", "float16"), ("float32", "float32")):
        store = _worker_store(se, value_dtype, se.Sgd(lr=1.0), dims=(2,), low=0.0, high=0.0,
                              gradient_dtype=gradient_dtype)
        store.lookup_or_insert(keys, 2)

        async def accumulate(store=store, gradient_dtype=gradient_dtype) -> np.ndarray:
            await store.async_accumulate_gradients(keys, np.asarray([[1.0, 2.0]], dtype=np.dtype(gradient_dtype)))
            await store.async_optimizer_step(1)
            values, _ = await store.async_lookup(keys, 2)
            return np.asarray(values)

        updated = asyncio.run(accumulate())
        assert store.value_dtype() == value_dtype
        assert store.optimizer_dtype() == "float32"
        assert updated.dtype == np.dtype(value_dtype)
        np.testing.assert_array_equal(updated, np.asarray([[-1.0, -2.0]], dtype=value_dtype))
    no_device_errors()


def test_flushed_partial_window(gpu_device, no_device_errors, se):
    """A window flushed after one micro-step is normalized by its actual length
    (test_checkpointing.py:229-251)."""
    store = _worker_store(se, "float32", se.Sgd(lr=1.0), dims=(2,), low=0.0, high=0.0)
    keys = np.asarray([7], dtype=np.int64)
    store.lookup_or_insert(keys, 2)
    store.accumulate_gradients(keys, np.asarray([[1.0, 1.0]], dtype=np.float32))
    asyncio.run(store.async_optimizer_step(1))
    values, _ = store.lookup(keys, 2)
    np.testing.assert_array_equal(np.asarray(values), [[-1.0, -1.0]])
    no_device_errors()


def test_adam_known_answer_through_the_worker_store(gpu_device, no_device_errors, se):
    """Zero init, Adam(lr=0.1), gradient ones: -0.1 after one step, -0.2 after two
    (tests/runtime/test_sparse_storage_limits.py:41-119)."""
    store = _worker_store(se, "float32", se.Adam(lr=0.1, dynamic_lr_policy=se.ConstantLrPolicy()), dims=(4,),
                          low=0.0, high=0.0)
    keys = np.asarray([11, 12], dtype=np.int64)
    store.lookup_or_insert(keys, 4)
    for expected in (-0.1, -0.2):
        store.accumulate_gradients(keys, np.ones((2, 4), np.float32))
        store.optimizer_step(1)
        values, _ = store.lookup(keys, 4)
        np.testing.assert_allclose(np.asarray(values), np.full((2, 4), expected), rtol=1e-5, atol=1e-6)
    no_device_errors()


def test_store_grows_past_its_initial_rows(gpu_device, no_device_errors, se):
    """Without reserve, lookup_or_insert grows the table (the reference's store pages in more rows)."""
    dim = 4
    cfg = se.EmbeddingConfig(dims=[dim], value_dtype="float32", key_dtype="int64")
    store = se.EmbeddingStore(embedding_config=cfg, optimizer_config=se.Sgd(lr=1.0), initial_rows=64)
    keys = np.arange(1000, dtype=np.int64) * 7919
    for lo in range(0, keys.size, 300):
        store.lookup_or_insert(keys[lo:lo + 300], dim)
    values, _ = store.lookup(keys, dim)
    np.testing.assert_array_equal(np.asarray(values), O.keymap_initial_values(keys, dim, -0.01, 0.01, 0, "float32"))
    assert store.size(dim) == keys.size
    no_device_errors()


def test_store_orders_inputs_from_another_stream(gpu_device, no_device_errors):
    """Keys and gradients written on the caller's stream behind a ~20 ms delaying kernel, results
    consumed on that stream: nothing calls synchronize() on the store."""
    from flare_amd.store import DynamicEmbeddingStore, Sgd, Uniform

    dim = 16
    store = DynamicEmbeddingStore(4096, [dim], value_dtype="float32", optimizer=Sgd(lr=1.0),
                                  initializer=Uniform(0.0, 0.0), seed=2)
    producer = torch.cuda.Stream(device=gpu_device)
    true_keys = torch.arange(100, 1100, dtype=torch.int64, device=gpu_device)
    keys = torch.full_like(true_keys, -5)
    grad = torch.zeros((1000, dim), dtype=torch.float32, device=gpu_device)
    torch.cuda.synchronize()
    with torch.cuda.stream(producer):
        torch.cuda._sleep(40_000_000)
        keys.copy_(true_keys)
        grad.fill_(2.0)
        values, _ = store.lookup_or_insert(keys, dim)
        rows = store.rows(keys, dim)
        store.accumulate_gradients(keys, grad)
        store.optimizer_step(1)
        after, _ = store.lookup(keys, dim)
        got_rows = rows.cpu()   # on the producer stream: waits for it, not for the store
        got_after = after.cpu()
        got_values = values.cpu()
    np.testing.assert_array_equal(got_rows.numpy(), np.arange(1000, dtype=np.int32))
    np.testing.assert_array_equal(got_values.numpy(), np.zeros((1000, dim), np.float32))
    np.testing.assert_array_equal(got_after.numpy(), np.full((1000, dim), -2.0, np.float32))
    no_device_errors()
