"""Gradient transport dtypes and the finite check, fused into the update.

The reference casts a bf16 / fp32 transport gradient to the fp32 native gradient before the
store accumulates it, and optionally rejects non-finite values
(sparse_precision.py:121-192, dynamic_embedding.py:508-513).  bf16 widens to fp32 exactly, so a
bf16 gradient read as it is must give the same bits as the cast-first path, and the update must
match the oracle run on the widened gradient; a rejected gradient must leave the table untouched.
The keyed sums the scatter hands back in the bf16 transport dtype (train_worker.py:518-522) are
the oracle's fp32 sums rounded to nearest even.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _host(t: torch.Tensor) -> np.ndarray:
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).cpu().numpy().view(np.uint16)
    return t.cpu().numpy()


def _shard(w, seed=3):
    from flare_amd.store import PooledTableShard, RowWiseAdagrad, Uniform

    return PooledTableShard(w.table_rows, w.dim, value_dtype=w.value_dtype, optimizer=RowWiseAdagrad(lr=0.01),
                            initializer=Uniform(-0.01, 0.01), seed=seed)


@pytest.mark.parametrize("config,batch,row_scale", [(2, 2048, 0.001), (4, 512, 0.0005), (3, 128, 0.0005)])
def test_bf16_pooled_gradient_equals_cast_first(gpu_device, no_device_errors, config, batch, row_scale):
    from flare_amd.workload import make_workload, pooled_grad_host

    w = make_workload(config, batch=batch, row_scale=row_scale)
    grad_bf16 = torch.from_numpy(pooled_grad_host(w) * np.float32(50)).to(gpu_device).to(torch.bfloat16)
    a, b = _shard(w), _shard(w)
    a.apply_pooled_gradients(w.ids, w.offsets, w.batch, grad_bf16, pooling=w.pooling, per_sample_weights=w.weights)
    b.apply_pooled_gradients(w.ids, w.offsets, w.batch, grad_bf16.to(torch.float32), pooling=w.pooling,
                             per_sample_weights=w.weights)
    a.synchronize()
    b.synchronize()
    np.testing.assert_array_equal(_host(a.table), _host(b.table))
    np.testing.assert_array_equal(a.state.state0.cpu().numpy(), b.state.state0.cpu().numpy())
    no_device_errors()


def test_plan_apply_bf16_and_validate(gpu_device, no_device_errors):
    from flare_amd.workload import make_workload, pooled_grad_host

    w = make_workload(2, batch=1024, row_scale=0.001)
    g = torch.from_numpy(pooled_grad_host(w)).to(gpu_device)
    a, b = _shard(w), _shard(w)
    pa = a.plan_step(w.ids, w.offsets, w.batch)
    pb = b.plan_step(w.ids, w.offsets, w.batch)
    pa.step(g.to(torch.bfloat16))
    pb.forward()
    pb.dedup()
    pb.apply(g.to(torch.bfloat16).to(torch.float32), validate_values=True)
    a.synchronize()
    b.synchronize()
    np.testing.assert_array_equal(_host(a.table), _host(b.table))
    assert int(pb.nonfinite.item()) == 0
    before = _host(a.table).copy()
    bad = g.clone()
    bad[3, 5, 7] = float("nan")
    with pytest.raises(FloatingPointError, match="non-finite sparse values"):
        pa.apply(bad, validate_values=True)
    np.testing.assert_array_equal(_host(a.table), before)
    no_device_errors(8)


@pytest.mark.parametrize("bad_value", [float("inf"), float("-inf"), float("nan")])
def test_pooled_validate_rejects_whole_batch(gpu_device, no_device_errors, bad_value):
    from flare_amd.workload import make_workload, pooled_grad_host

    w = make_workload(4, batch=300, row_scale=0.0005)
    shard = _shard(w)
    grad = pooled_grad_host(w)
    grad[-1, -1, -1] = bad_value  # the very last element
    before = _host(shard.table).copy()
    acc = shard.state.state0.cpu().numpy().copy()
    with pytest.raises(FloatingPointError):
        shard.apply_pooled_gradients(w.ids, w.offsets, w.batch, grad, validate_values=True)
    np.testing.assert_array_equal(_host(shard.table), before)
    np.testing.assert_array_equal(shard.state.state0.cpu().numpy(), acc)
    no_device_errors(8)
    grad[-1, -1, -1] = 0.0
    shard.apply_pooled_gradients(w.ids, w.offsets, w.batch, grad, validate_values=True)
    shard.synchronize()
    assert not np.array_equal(_host(shard.table), before)
    no_device_errors()


@pytest.mark.parametrize("value_dtype", ["float32", "bfloat16"])
def test_store_bf16_gradients_equal_cast_first(gpu_device, no_device_errors, value_dtype):
    from flare_amd.store import Adam, EmbeddingStore

    rng = np.random.default_rng(4)
    stores = [EmbeddingStore(capacity=2000, dims=[64], value_dtype=value_dtype, optimizer=Adam(lr=0.01), seed=9)
              for _ in range(2)]
    for _ in range(2):
        keys = rng.integers(0, 2000, 3000).astype(np.int64)
        g = torch.from_numpy(rng.standard_normal((3000, 64), dtype=np.float32)).to(gpu_device).to(torch.bfloat16)
        stores[0].accumulate_gradients(keys, g)
        stores[1].accumulate_gradients(keys, g.to(torch.float32))
    for s in stores:
        s.optimizer_step(2)
        s.synchronize()
    np.testing.assert_array_equal(_host(stores[0].tables[64].table), _host(stores[1].tables[64].table))
    np.testing.assert_array_equal(stores[0].tables[64].state0.cpu().numpy(), stores[1].tables[64].state0.cpu().numpy())
    no_device_errors()


def test_store_validate_raises_before_accumulating(gpu_device, no_device_errors):
    from flare_amd.store import EmbeddingStore, Sgd, Zeros

    store = EmbeddingStore(capacity=16, dims=[4], value_dtype="float32", optimizer=Sgd(lr=1.0),
                           initializer=Zeros(), validate_values=True)
    keys = np.asarray([1, 2], np.int64)
    with pytest.raises(FloatingPointError, match="non-finite sparse values at sparse_native_gradient"):
        store.accumulate_gradients(keys, np.asarray([[1, 2, 3, 4], [1, np.inf, 3, 4]], np.float32))
    no_device_errors(8)
    store.accumulate_gradients(keys, np.ones((2, 4), np.float32))
    store.optimizer_step(1)
    values, _ = store.lookup(keys, 4)
    store.synchronize()
    np.testing.assert_array_equal(values.cpu().numpy(), -np.ones((2, 4), np.float32))
    no_device_errors()


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_check_finite_every_position(gpu_device, no_device_errors, dtype):
    from flare_amd import _native
    from flare_amd.conversion import storage_code

    flag = torch.empty(1, dtype=torch.int32, device=gpu_device)
    for count in (1, 7, 8, 9, 1000, 4099):
        for offset in (0, 1):  # 16-byte aligned and not
            base = torch.zeros(count + offset, dtype=dtype, device=gpu_device)
            view = base[offset:]
            _native.call("flare_check_finite", view.data_ptr(), storage_code(dtype), count, flag.data_ptr(), None)
            torch.cuda.synchronize()
            assert int(flag.item()) == 0
            for pos in sorted({0, count // 2, count - 1}):
                for bad in (float("inf"), float("nan")):
                    view.zero_()
                    view[pos] = bad
                    _native.call("flare_check_finite", view.data_ptr(), storage_code(dtype), count, flag.data_ptr(),
                                 None)
                    torch.cuda.synchronize()
                    assert int(flag.item()) == 1, (count, offset, pos, bad)
    no_device_errors(8)
    view = torch.full((33,), 65504.0, dtype=torch.float32, device=gpu_device)  # large but finite
    _native.call("flare_check_finite", view.data_ptr(), storage_code(torch.float32), 33, flag.data_ptr(), None)
    torch.cuda.synchronize()
    assert int(flag.item()) == 0
    no_device_errors()


@pytest.mark.parametrize("config,batch,row_scale", [(2, 2048, 0.001), (4, 512, 0.0005), (5, 96, 0.00005)])
def test_bf16_pooled_gradient_matches_oracle(gpu_device, no_device_errors, config, batch, row_scale):
    """The update read from a bf16 pooled gradient against the oracle run on that gradient widened
    to fp32 (prepare_sparse_native_gradient's cast, sparse_precision.py:150-192)."""
    from flare_amd.store import Adam, PooledTableShard, RowWiseAdagrad, Uniform
    from flare_amd.workload import make_workload, pooled_grad_host
    from oracle import sparse_oracle as O

    w = make_workload(config, batch=batch, row_scale=row_scale)
    adam = w.optimizer == "adam"
    shard = PooledTableShard(w.table_rows, w.dim, value_dtype=w.value_dtype,
                             optimizer=Adam(lr=0.01) if adam else RowWiseAdagrad(lr=0.01),
                             initializer=Uniform(-0.01, 0.01), seed=5)
    table0 = _host(shard.table.clone())
    grad_bf16 = torch.from_numpy(pooled_grad_host(w) * np.float32(30)).to(gpu_device).to(torch.bfloat16)
    unique, inverse, first = shard.apply_pooled_gradients(w.ids, w.offsets, w.batch, grad_bf16, pooling=w.pooling,
                                                          per_sample_weights=w.weights, return_dedup=True)
    shard.synchronize()
    state = ({"m": np.zeros((w.total_rows, w.dim), np.float32), "v": np.zeros((w.total_rows, w.dim), np.float32),
              "step": np.zeros(w.total_rows, np.int32)} if adam else {"acc": np.zeros(w.total_rows, np.float32)})
    _, e_table, e_state, e_unique, e_inverse, e_first = O.pooled_step(
        table0, state, w.ids, w.offsets, w.row_base(), w.batch, w.dim, grad_bf16.to(torch.float32).cpu().numpy(),
        storage=w.value_dtype, pooling=w.pooling, weights=w.weights, optimizer="adam" if adam else "rowwise_adagrad")
    np.testing.assert_array_equal(unique.cpu().numpy(), e_unique)
    np.testing.assert_array_equal(inverse.cpu().numpy(), e_inverse)
    np.testing.assert_array_equal(first.cpu().numpy(), e_first)
    assert O.storage_ulp_distance(_host(shard.table), e_table, w.value_dtype).max() <= 1
    if adam:
        np.testing.assert_allclose(shard.state.state0.cpu().numpy(), e_state["m"], rtol=1e-5, atol=1e-12)
        np.testing.assert_allclose(shard.state.state1.cpu().numpy(), e_state["v"], rtol=1e-5, atol=1e-15)
    else:
        np.testing.assert_allclose(shard.state.state0.cpu().numpy(), e_state["acc"], rtol=1e-5, atol=0)
    no_device_errors()


@pytest.mark.parametrize("value_dtype", ["float32", "bfloat16"])
def test_store_bf16_gradients_match_oracle(gpu_device, no_device_errors, value_dtype):
    """accumulate_gradients with bf16 gradients over two micro-steps, optimizer_step(2), against
    the oracle's keyed sums of the widened gradients, divided by 2, and its Adam."""
    from flare_amd.store import Adam, EmbeddingStore
    from oracle import sparse_oracle as O

    rng = np.random.default_rng(12)
    rows, dim = 1500, 32
    store = EmbeddingStore(capacity=rows, dims=[dim], value_dtype=value_dtype, optimizer=Adam(lr=0.01), seed=4)
    table0 = _host(store.tables[dim].table.clone())
    all_keys, all_grads = [], []
    for _ in range(2):
        keys = rng.integers(0, rows, 2500).astype(np.int64)
        g = torch.from_numpy(rng.standard_normal((2500, dim), dtype=np.float32)).to(gpu_device).to(torch.bfloat16)
        store.accumulate_gradients(keys, g)
        all_keys.append(keys)
        all_grads.append(g.to(torch.float32).cpu().numpy())
    store.optimizer_step(2)
    store.synchronize()
    keys = np.concatenate(all_keys)
    sums = O.scatter(rows, dim, keys, -1, np.concatenate(all_grads))
    touched = np.unique(keys)
    g = (sums[touched] / np.float32(2)).astype(np.float32)
    w0 = O.storage_to_f32(table0[touched], value_dtype)
    w1, m1, v1, s1 = O.adam_update(w0, np.zeros_like(g), np.zeros_like(g), np.zeros(touched.size, np.int32), g,
                                   lr=0.01)
    got = _host(store.tables[dim].table)[touched]
    assert O.storage_ulp_distance(got, O.f32_to_storage(w1, value_dtype), value_dtype).max() <= 1
    np.testing.assert_allclose(store.tables[dim].state0.cpu().numpy()[touched], m1, rtol=1e-5, atol=1e-12)
    np.testing.assert_array_equal(store.tables[dim].step.cpu().numpy()[touched], s1)
    no_device_errors()


@pytest.mark.parametrize("pooled", [True, False])
def test_scatter_in_transport_dtype_matches_oracle(gpu_device, no_device_errors, pooled):
    """Keyed sums stored as bf16 by the scatter itself: RNE of the oracle's fp32 sums, bit for bit,
    and the same bits as the caller's separate grad.astype('bfloat16')."""
    from flare_amd.operator import HipSparseEmbeddingOperator
    from oracle import sparse_oracle as O

    op = HipSparseEmbeddingOperator("float32", "float32", empty_cache=False)
    rng = np.random.default_rng(93)
    batch, features, max_el, dim, rows = 48, 12, 30, 128, 256
    inverse = rng.integers(0, rows + 1, size=(batch, features, max_el)).astype(np.int32)
    inverse[rng.random(inverse.shape) < 0.5] = rows  # pad slots
    grad = rng.normal(0, 1, size=(batch, features, dim)).astype(np.float32)
    if pooled:
        fused = op.scatter_pooled(rows, dim, inverse, rows, grad, (features, max_el), out_dtype="bfloat16")
        plain = op.scatter_pooled(rows, dim, inverse, rows, grad, (features, max_el))
        expected = O.scatter_pooled(rows, dim, inverse, rows, grad, (features, max_el))
    else:
        slot_grad = grad.reshape(-1, dim)[np.arange(inverse.size) // max_el]
        fused = op.scatter(rows, dim, inverse.reshape(-1), rows, slot_grad, out_dtype="bfloat16")
        plain = op.scatter(rows, dim, inverse.reshape(-1), rows, slot_grad)
        expected = O.scatter(rows, dim, inverse.reshape(-1), rows, slot_grad)
    cast = plain.astype("bfloat16")
    op.stream.synchronize()
    assert fused.tensor.dtype == torch.bfloat16 and tuple(fused.shape) == (rows, dim)
    np.testing.assert_array_equal(_host(fused.tensor), O.f32_to_bf16_bits(expected))
    np.testing.assert_array_equal(_host(cast.tensor), O.f32_to_bf16_bits(expected))
    no_device_errors()
