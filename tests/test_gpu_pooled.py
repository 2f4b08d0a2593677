"""Fused CSR path on the GPU: pooled lookup and pooled-gradient update vs the oracle.

Small-scale versions of the five workloads (same generators, fewer rows and
samples) are compared against ``oracle.sparse_oracle.pooled_step``:
pooled outputs bit-exact (same fp32 order, RNE), unique / inverse /
first_indices bit-exact, optimizer state within rtol 1e-5 and stored rows
within 1 ulp of the storage dtype.
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


def _shard(w, optimizer, seed=3):
    from flare_amd.store import Adam, PooledTableShard, RowWiseAdagrad, Sgd, Uniform

    opt = {"rowwise_adagrad": RowWiseAdagrad(lr=0.01, eps=1e-8), "adam": Adam(lr=0.01),
           "sgd": Sgd(lr=0.01), "none": RowWiseAdagrad()}[optimizer]
    return PooledTableShard(w.table_rows, w.dim, value_dtype=w.value_dtype, optimizer=opt,
                            initializer=Uniform(-w.init_range, w.init_range), seed=seed)


CASES = [
    # config, batch, row_scale, optimizer override
    (1, 512, 0.01, None),
    (2, 2048, 0.001, None),
    (3, 256, 0.0005, "rowwise_adagrad"),
    (4, 1024, 0.0005, None),
    (5, 256, 0.00005, None),
    (2, 700, 0.0001, "sgd"),
    (4, 300, 0.0002, "adam"),
]


@pytest.mark.parametrize("case", range(len(CASES)))
def test_pooled_step_matches_oracle(gpu_device, no_device_errors, case):
    from flare_amd.workload import make_workload, pooled_grad_host

    config, batch, row_scale, override = CASES[case]
    w = make_workload(config, batch=batch, row_scale=row_scale)
    optimizer = override or w.optimizer
    if optimizer == "none":
        optimizer = "rowwise_adagrad"
    shard = _shard(w, optimizer)
    table0 = _host(shard.table.clone())
    grad = pooled_grad_host(w)
    pooled = shard.lookup_pooled(w.ids, w.offsets, w.batch, pooling=w.pooling, per_sample_weights=w.weights)
    dedup = shard.apply_pooled_gradients(w.ids, w.offsets, w.batch, grad, pooling=w.pooling,
                                         per_sample_weights=w.weights, return_dedup=True)
    shard.synchronize()
    state = {}
    if optimizer == "rowwise_adagrad":
        state = {"acc": np.zeros(w.total_rows, np.float32)}
    elif optimizer == "adam":
        state = {"m": np.zeros((w.total_rows, w.dim), np.float32), "v": np.zeros((w.total_rows, w.dim), np.float32),
                 "step": np.zeros(w.total_rows, np.int32)}
    e_pooled, e_table, e_state, e_unique, e_inverse, e_first = O.pooled_step(
        table0, state, w.ids, w.offsets, w.row_base(), w.batch, w.dim, grad,
        storage=w.value_dtype, pooling=w.pooling, weights=w.weights, optimizer=optimizer)
    np.testing.assert_array_equal(_host(pooled), e_pooled)
    unique, inverse, first = (t.cpu().numpy() for t in dedup)
    np.testing.assert_array_equal(unique, e_unique)
    np.testing.assert_array_equal(inverse, e_inverse)
    np.testing.assert_array_equal(first, e_first)
    got = _host(shard.table)
    ulps = O.storage_ulp_distance(got, e_table, w.value_dtype)
    assert ulps.max() <= 1, f"max ulp {ulps.max()} over {np.count_nonzero(ulps)} elements"
    if optimizer == "rowwise_adagrad":
        np.testing.assert_allclose(shard.state.state0.cpu().numpy(), e_state["acc"], rtol=1e-5, atol=0)
    elif optimizer == "adam":
        np.testing.assert_allclose(shard.state.state0.cpu().numpy(), e_state["m"], rtol=1e-5, atol=1e-12)
        np.testing.assert_allclose(shard.state.state1.cpu().numpy(), e_state["v"], rtol=1e-5, atol=1e-15)
        np.testing.assert_array_equal(shard.state.step.cpu().numpy(), e_state["step"])
    no_device_errors()


@pytest.mark.parametrize("pooling", ["weighted", "mean", "sum"])
def test_reduced_gradients_bit_exact(gpu_device, no_device_errors, pooling):
    """Backward-only (workload 3 form): per-key gradients in first-occurrence order."""
    from flare_amd.workload import make_workload, pooled_grad_host

    w = make_workload(3, batch=300, row_scale=0.0002)
    shard = _shard(w, "rowwise_adagrad")
    grad = pooled_grad_host(w)
    pooled = shard.lookup_pooled(w.ids, w.offsets, w.batch, pooling=pooling, per_sample_weights=w.weights)
    unique, inverse, first, g = shard.reduce_pooled_gradients(w.ids, w.offsets, w.batch, grad, pooling=pooling,
                                                              per_sample_weights=w.weights)
    shard.synchronize()
    eu, ei, ef, eg = O.pooled_grad_sums(w.ids, w.offsets, w.row_base(), w.batch, w.dim, grad,
                                        pooling=pooling, weights=w.weights)
    np.testing.assert_array_equal(unique.cpu().numpy(), eu)
    np.testing.assert_array_equal(inverse.cpu().numpy(), ei)
    np.testing.assert_array_equal(first.cpu().numpy(), ef)
    np.testing.assert_array_equal(g.cpu().numpy(), eg)
    ep = O.gather_pooled_csr(_host(shard.table), w.ids, w.offsets, w.row_base(), w.batch, w.dim,
                             storage=w.value_dtype, pooling=pooling, weights=w.weights)
    np.testing.assert_array_equal(_host(pooled), ep)
    no_device_errors()


def test_overlapped_step_plan_matches_oracle(gpu_device, no_device_errors):
    """PooledStepPlan.step: dedup on a second stream concurrent with the forward."""
    from flare_amd.workload import make_workload, pooled_grad_host

    w = make_workload(2, batch=3000, row_scale=0.0005)
    shard = _shard(w, "rowwise_adagrad")
    table0 = _host(shard.table.clone())
    grad = torch.from_numpy(pooled_grad_host(w)).to(gpu_device)
    plan = shard.plan_step(w.ids, w.offsets, w.batch)
    state = {"acc": np.zeros(w.total_rows, np.float32)}
    table = table0
    for _ in range(2):  # the second step reads rows the first one updated
        pooled = plan.step(grad)
        shard.synchronize()
        e_pooled, table, state, e_unique, e_inverse, e_first = O.pooled_step(
            table, state, w.ids, w.offsets, w.row_base(), w.batch, w.dim, grad.cpu().numpy(),
            storage=w.value_dtype)
        np.testing.assert_array_equal(_host(pooled), e_pooled)
        u = int(plan.unique_count.item())
        np.testing.assert_array_equal(plan.unique[:u].cpu().numpy(), e_unique)
        np.testing.assert_array_equal(plan.first_indices[:u].cpu().numpy(), e_first)
        np.testing.assert_array_equal(plan.inverse[:w.num_ids].cpu().numpy(), e_inverse)
        ulps = O.storage_ulp_distance(_host(shard.table), table, w.value_dtype)
        assert ulps.max() <= 1
        table = _host(shard.table)  # continue from the device state (ulp-level ties)
        state = {"acc": shard.state.state0.cpu().numpy()}
    no_device_errors()


RAGGED = [
    # batch, dim, max bag length (bags of length 0 included)
    (1, 128, 9),     # each group of four bags spans four tables
    (3, 24, 70),     # bags longer than one id chunk; 3-vector rows
    (7, 20, 5),      # dim not a multiple of the 16-byte vector: scalar lanes
    (130, 300, 3),   # fp32 rows of 300 (two vectors per lane)
    (5, 1100, 4),    # several column passes
    (257, 64, 40),   # long bags (one bag per lane group, 8 rows in flight), partial last block
]


@pytest.mark.parametrize("storage", ["bfloat16", "float16", "float32"])
@pytest.mark.parametrize("pooling", ["sum", "mean", "weighted"])
@pytest.mark.parametrize("case", range(len(RAGGED)))
def test_csr_ragged_bags_bit_exact(gpu_device, no_device_errors, storage, pooling, case):
    """Empty bags, bags spanning id chunks and tables, every row shape: forward and reduced grads."""
    from flare_amd.store import PooledTableShard, Uniform

    batch, dim, max_len = RAGGED[case]
    rng = np.random.default_rng(100 + case)
    table_rows = [5, 40, 17]
    lengths = rng.integers(0, max_len + 1, size=len(table_rows) * batch)
    lengths[::4] = 0
    offsets = np.zeros(lengths.size + 1, np.int64)
    offsets[1:] = np.cumsum(lengths)
    bag_table = np.repeat(np.arange(lengths.size) // batch, lengths)
    ids = (rng.integers(0, 1 << 30, size=int(offsets[-1])) % np.asarray(table_rows)[bag_table]).astype(np.int64)
    weights = rng.uniform(0, 1, size=ids.size).astype(np.float32)
    shard = PooledTableShard(table_rows, dim, value_dtype=storage, initializer=Uniform(-1.0, 1.0), seed=case)
    row_base = np.concatenate([[0], np.cumsum(table_rows)]).astype(np.int64)
    w = weights if pooling == "weighted" else None
    pooled = shard.lookup_pooled(ids, offsets, batch, pooling=pooling, per_sample_weights=w)
    grad = rng.normal(0, 1, size=(batch, len(table_rows), dim)).astype(np.float32)
    unique, inverse, first, g = shard.reduce_pooled_gradients(ids, offsets, batch, grad, pooling=pooling,
                                                              per_sample_weights=w)
    shard.synchronize()
    expected = O.gather_pooled_csr(_host(shard.table), ids, offsets, row_base, batch, dim, storage=storage,
                                   pooling=pooling, weights=w)
    np.testing.assert_array_equal(_host(pooled), expected)
    eu, ei, ef, eg = O.pooled_grad_sums(ids, offsets, row_base, batch, dim, grad, pooling=pooling, weights=w)
    np.testing.assert_array_equal(unique.cpu().numpy(), eu)
    np.testing.assert_array_equal(inverse.cpu().numpy(), ei)
    np.testing.assert_array_equal(first.cpu().numpy(), ef)
    np.testing.assert_array_equal(g.cpu().numpy(), eg)
    no_device_errors()


def test_shard_with_25_bit_rows(gpu_device, no_device_errors):
    """Tables totalling 2^25 rows: 25-bit row keys (three 9-bit radix passes) on the CSR path."""
    from flare_amd.store import PooledTableShard, Uniform

    rng = np.random.default_rng(25)
    table_rows = [1 << 24, (1 << 24) - 1000, 1000]
    batch, dim = 4096, 4
    lengths = rng.integers(0, 4, size=len(table_rows) * batch)
    offsets = np.zeros(lengths.size + 1, np.int64)
    offsets[1:] = np.cumsum(lengths)
    bag_table = np.repeat(np.arange(lengths.size) // batch, lengths)
    ids = (rng.integers(0, 1 << 40, size=int(offsets[-1])) % np.asarray(table_rows)[bag_table]).astype(np.int64)
    ids[rng.random(ids.size) < 0.2] = 0  # hot first rows
    shard = PooledTableShard(table_rows, dim, value_dtype="float32", initializer=Uniform(-1.0, 1.0), seed=3)
    row_base = np.concatenate([[0], np.cumsum(table_rows)]).astype(np.int64)
    pooled = shard.lookup_pooled(ids, offsets, batch)
    grad = rng.normal(0, 1, size=(batch, len(table_rows), dim)).astype(np.float32)
    unique, inverse, first, g = shard.reduce_pooled_gradients(ids, offsets, batch, grad)
    shard.synchronize()
    expected = O.gather_pooled_csr(shard.table.cpu().numpy(), ids, offsets, row_base, batch, dim)
    np.testing.assert_array_equal(pooled.cpu().numpy(), expected)
    eu, ei, ef, eg = O.pooled_grad_sums(ids, offsets, row_base, batch, dim, grad)
    np.testing.assert_array_equal(unique.cpu().numpy(), eu)
    np.testing.assert_array_equal(inverse.cpu().numpy(), ei)
    np.testing.assert_array_equal(first.cpu().numpy(), ef)
    np.testing.assert_array_equal(g.cpu().numpy(), eg)
    no_device_errors()


@pytest.mark.parametrize("case", [(2, 2048, 0.001, "sum"), (4, 1024, 0.0005, "mean"), (3, 256, 0.0005, "weighted"),
                                  (1, 512, 0.01, "sum")])
def test_plan_forward_dedup_apply(gpu_device, no_device_errors, case):
    """PooledStepPlan: forward(), dedup(), apply() in turn on one stream, two steps (sum, mean, weighted)."""
    from flare_amd.workload import make_workload, pooled_grad_host

    config, batch, row_scale, pooling = case
    w = make_workload(config, batch=batch, row_scale=row_scale)
    shard = _shard(w, "rowwise_adagrad")
    table0 = _host(shard.table.clone())
    weights = w.weights if pooling == "weighted" else None
    if pooling == "weighted" and weights is None:
        weights = np.random.default_rng(4).uniform(0, 1, w.num_ids).astype(np.float32)
    plan = shard.plan_step(w.ids, w.offsets, w.batch, pooling=pooling, per_sample_weights=weights)
    grad = torch.from_numpy(pooled_grad_host(w)).to(gpu_device)
    state = {"acc": np.zeros(w.total_rows, np.float32)}
    table = table0
    for _ in range(2):
        pooled = plan.forward()
        plan.dedup()
        plan.apply(grad)
        shard.synchronize()
        e_pooled, table, state, e_unique, e_inverse, e_first = O.pooled_step(
            table, state, w.ids, w.offsets, w.row_base(), w.batch, w.dim, grad.cpu().numpy(),
            storage=w.value_dtype, pooling=pooling, weights=weights)
        np.testing.assert_array_equal(_host(pooled), e_pooled)
        u = int(plan.unique_count.item())
        np.testing.assert_array_equal(plan.unique[:u].cpu().numpy(), e_unique)
        np.testing.assert_array_equal(plan.first_indices[:u].cpu().numpy(), e_first)
        np.testing.assert_array_equal(plan.inverse[:w.num_ids].cpu().numpy(), e_inverse)
        assert O.storage_ulp_distance(_host(shard.table), table, w.value_dtype).max() <= 1
        np.testing.assert_allclose(shard.state.state0.cpu().numpy(), state["acc"], rtol=1e-5, atol=0)
        table = _host(shard.table)
        state = {"acc": shard.state.state0.cpu().numpy()}
    no_device_errors()


def test_forward_reports_invalid_offsets(gpu_device, no_device_errors):
    """Decreasing or out-of-range CSR offsets pool nothing out of range and set the error bit
    (the reference validates offsets, recipes/recsys/ranking/schema/input.py:96-114)."""
    from flare_amd.store import PooledTableShard

    shard = PooledTableShard([10, 10], 4, value_dtype="float32")
    ids = np.asarray([1, 2, 3, 4], np.int64)
    good = np.asarray([0, 1, 2, 3, 4], np.int64)
    shard.lookup_pooled(ids, good, 2)
    no_device_errors(0)
    for bad in (np.asarray([0, 3, 1, 3, 4], np.int64),    # decreasing
                np.asarray([0, 1, 2, 3, 9], np.int64),    # past the ids
                np.asarray([1, 1, 2, 3, 4], np.int64)):   # not starting at 0
        out = shard.lookup_pooled(ids, bad, 2)
        shard.synchronize()
        assert np.isfinite(out.cpu().numpy()).all()
        no_device_errors(1)



def test_backward_rejects_invalid_offsets(gpu_device, no_device_errors):
    """A batch whose CSR offsets fail validation updates nothing, reports no unique ids and sets
    the error bit, after a valid batch has left its sort in the workspace (the reference
    validates offsets before use, recipes/recsys/ranking/schema/input.py:96-114)."""
    from flare_amd.store import PooledTableShard

    shard = PooledTableShard([10, 10], 4, value_dtype="float32", seed=3)
    ids = np.asarray([1, 2, 3, 4], np.int64)
    good = np.asarray([0, 1, 2, 3, 4], np.int64)
    grad = np.ones((2, 2, 4), np.float32)
    shard.apply_pooled_gradients(ids, good, 2, grad)
    shard.synchronize()
    no_device_errors(0)
    table = _host(shard.table.clone())
    acc = shard.state.state0.cpu().numpy().copy()
    for bad in (np.asarray([0, 3, 1, 3, 4], np.int64),    # decreasing
                np.asarray([0, 1, 2, 3, 9], np.int64),    # past the ids
                np.asarray([1, 1, 2, 3, 4], np.int64)):   # not starting at 0
        unique, inverse, first = shard.apply_pooled_gradients(ids, bad, 2, grad, return_dedup=True)
        shard.synchronize()
        assert unique.numel() == 0 and first.numel() == 0
        np.testing.assert_array_equal(_host(shard.table), table)
        np.testing.assert_array_equal(shard.state.state0.cpu().numpy(), acc)
        no_device_errors(1)
    shard.apply_pooled_gradients(ids, good, 2, grad)  # the next valid batch is applied
    shard.synchronize()
    no_device_errors(0)
    assert not np.array_equal(_host(shard.table), table)

@pytest.mark.parametrize("case", ["long_bags_listed", "more_long_bags_than_the_list"])
def test_short_bag_prepare_with_long_bags(gpu_device, no_device_errors, case):
    """Batches averaging at most 8 ids per bag take the per-bag walk in the dedup's prepare;
    its long bags go to a block-wide walk, and past 256 of them in a block to their own thread."""
    from flare_amd.store import PooledTableShard, Uniform

    rng = np.random.default_rng(31)
    if case == "long_bags_listed":
        table_rows, batch, dim = [20, 35, 7], 2000, 16
        lengths = rng.integers(0, 3, size=len(table_rows) * batch)
        lengths[::50] = 200
    else:
        table_rows, batch, dim = [50], 600000, 8
        lengths = rng.integers(0, 2, size=batch)
        lengths[:1200:4] = 33  # 300 long bags inside the first prepare block
    assert lengths.sum() <= 8 * lengths.size
    offsets = np.zeros(lengths.size + 1, np.int64)
    offsets[1:] = np.cumsum(lengths)
    bag_table = np.repeat(np.arange(lengths.size) // batch, lengths)
    ids = (rng.integers(0, 1 << 30, size=int(offsets[-1])) % np.asarray(table_rows)[bag_table]).astype(np.int64)
    shard = PooledTableShard(table_rows, dim, value_dtype="float32", initializer=Uniform(-1.0, 1.0), seed=4)
    row_base = np.concatenate([[0], np.cumsum(table_rows)]).astype(np.int64)
    grad = rng.normal(0, 1, size=(batch, len(table_rows), dim)).astype(np.float32)
    unique, inverse, first, g = shard.reduce_pooled_gradients(ids, offsets, batch, grad)
    shard.synchronize()
    eu, ei, ef, eg = O.pooled_grad_sums(ids, offsets, row_base, batch, dim, grad)
    np.testing.assert_array_equal(unique.cpu().numpy(), eu)
    np.testing.assert_array_equal(inverse.cpu().numpy(), ei)
    np.testing.assert_array_equal(first.cpu().numpy(), ef)
    np.testing.assert_array_equal(g.cpu().numpy(), eg)
    no_device_errors()


def test_pooled_step_with_a_key_past_the_fold_chunk(gpu_device, no_device_errors):
    """Row-wise Adagrad through the fused path when one key holds ~60% of 20K occurrences."""
    from flare_amd.store import PooledTableShard, RowWiseAdagrad, Uniform

    rng = np.random.default_rng(41)
    table_rows, batch, dim = [30, 9], 10000, 64
    ids = rng.integers(0, 9, size=2 * batch).astype(np.int64)
    ids[:batch][rng.random(batch) < 0.6] = 4   # hot key of table 0: ~6K occurrences, ~94 units
    ids[:batch] = np.where(ids[:batch] < 30, ids[:batch], 0)
    offsets = np.arange(2 * batch + 1, dtype=np.int64)
    shard = PooledTableShard(table_rows, dim, value_dtype="float32", optimizer=RowWiseAdagrad(lr=0.01),
                             initializer=Uniform(-1.0, 1.0), seed=8)
    table0 = shard.table.clone().cpu().numpy()
    grad = rng.normal(0, 1e-2, size=(batch, 2, dim)).astype(np.float32)
    shard.apply_pooled_gradients(ids, offsets, batch, grad)
    shard.synchronize()
    row_base = np.asarray([0, 30, 39], np.int64)
    _, e_table, e_state, *_ = O.pooled_step(table0, {"acc": np.zeros(39, np.float32)}, ids, offsets, row_base,
                                             batch, dim, grad, storage="float32")
    assert O.storage_ulp_distance(shard.table.cpu().numpy(), e_table, "float32").max() <= 1
    np.testing.assert_allclose(shard.state.state0.cpu().numpy(), e_state["acc"], rtol=1e-5)
    no_device_errors()


# 16-byte vectors per row: 8, 16, 32 (one per lane), 4 (the narrowest group) and 128 (two per lane)
SHORT_DIMS = {"bfloat16": (64, 128, 256, 32, 1024), "float16": (64, 128, 256, 32, 1024),
              "float32": (32, 64, 128, 16, 512)}


@pytest.mark.parametrize("layout", ["sample_major", "table_major"])
@pytest.mark.parametrize("pooling", ["sum", "mean", "weighted"])
@pytest.mark.parametrize("storage", ["bfloat16", "float16", "float32"])
@pytest.mark.parametrize("width", [0, 1, 2, 3, 4])
def test_short_bag_forward_bit_exact(gpu_device, no_device_errors, layout, pooling, storage, width):
    """Bags of 0-2 ids (at most 2 on average, a few of 3-5), rows of 4 to 128 16-byte vectors,
    int32 and int64 ids, both pooled row layouts: the forward against the oracle."""
    from flare_amd.store import PooledTableShard, Uniform

    dim = SHORT_DIMS[storage][width]
    rng = np.random.default_rng(7 + width)
    table_rows, batch = [9, 300, 41], 777
    lengths = rng.integers(0, 3, size=len(table_rows) * batch)
    lengths[5::97] = rng.integers(3, 6, size=lengths[5::97].size)
    lengths[: lengths.size // 8] = np.minimum(lengths[: lengths.size // 8], 1)
    assert lengths.sum() <= 2 * lengths.size
    offsets = np.zeros(lengths.size + 1, np.int64)
    offsets[1:] = np.cumsum(lengths)
    bag_table = np.repeat(np.arange(lengths.size) // batch, lengths)
    ids = (rng.integers(0, 1 << 30, size=int(offsets[-1])) % np.asarray(table_rows)[bag_table]).astype(np.int64)
    weights = rng.uniform(0, 1, size=ids.size).astype(np.float32) if pooling == "weighted" else None
    shard = PooledTableShard(table_rows, dim, value_dtype=storage, initializer=Uniform(-1.0, 1.0), seed=width,
                             layout=layout)
    row_base = np.concatenate([[0], np.cumsum(table_rows)]).astype(np.int64)
    pooled = shard.lookup_pooled(ids.astype(np.int32) if width == 1 else ids, offsets, batch, pooling=pooling,
                                 per_sample_weights=weights)
    shard.synchronize()
    expected = O.gather_pooled_csr(_host(shard.table), ids, offsets, row_base, batch, dim, storage=storage,
                                   pooling=pooling, weights=weights)
    if layout == "table_major":
        expected = np.ascontiguousarray(expected.transpose(1, 0, 2))
    assert tuple(pooled.shape) == shard.pooled_shape(batch)
    np.testing.assert_array_equal(_host(pooled), expected)
    no_device_errors()


@pytest.mark.parametrize("pooling", ["sum", "mean"])
def test_short_bag_forward_skips_invalid_ids(gpu_device, no_device_errors, pooling):
    """Short bags with some ids past their table: those ids pool nothing (nor count for the
    mean) and set the error bit; every row equals the oracle's pooling of the valid ids."""
    from flare_amd.store import PooledTableShard, Uniform

    rng = np.random.default_rng(23)
    table_rows, batch, dim = [50, 7, 300], 400, 128
    lengths = rng.integers(0, 3, size=len(table_rows) * batch)
    offsets = np.zeros(lengths.size + 1, np.int64)
    offsets[1:] = np.cumsum(lengths)
    bag_table = np.repeat(np.arange(lengths.size) // batch, lengths)
    limit = np.asarray(table_rows)[bag_table]
    ids = rng.integers(0, 1 << 20, size=int(offsets[-1])) % limit
    bad = np.zeros(ids.size, bool)
    bad[3::37] = True
    ids = np.where(bad, limit + rng.integers(0, 5, size=ids.size), ids).astype(np.int64)
    shard = PooledTableShard(table_rows, dim, value_dtype="bfloat16", initializer=Uniform(-1.0, 1.0), seed=2,
                             layout="table_major")
    pooled = shard.lookup_pooled(ids, offsets, batch, pooling=pooling)
    shard.synchronize()
    keep_len = np.add.reduceat(~bad, offsets[:-1]) * (lengths > 0)
    keep_off = np.zeros(lengths.size + 1, np.int64)
    keep_off[1:] = np.cumsum(keep_len)
    row_base = np.concatenate([[0], np.cumsum(table_rows)]).astype(np.int64)
    expected = O.gather_pooled_csr(_host(shard.table), ids[~bad], keep_off, row_base, batch, dim,
                                   storage="bfloat16", pooling=pooling)
    np.testing.assert_array_equal(_host(pooled), np.ascontiguousarray(expected.transpose(1, 0, 2)))
    no_device_errors(1)


@pytest.mark.parametrize("config", [2, 4])
def test_table_major_step_matches_sample_major(gpu_device, no_device_errors, config):
    """The same step in both pooled row layouts: forward rows transposed, dedup identical, and the
    same table update (the [T, B, D] gradient is the [B, T, D] one transposed)."""
    from flare_amd.workload import make_workload, pooled_grad_host

    w = make_workload(config, batch=1500, row_scale=0.0005)
    grad = pooled_grad_host(w)
    results = {}
    for layout in ("sample_major", "table_major"):
        from flare_amd.store import PooledTableShard, RowWiseAdagrad, Uniform

        shard = PooledTableShard(w.table_rows, w.dim, value_dtype=w.value_dtype, optimizer=RowWiseAdagrad(),
                                 initializer=Uniform(-0.01, 0.01), seed=5, layout=layout)
        g = grad if layout == "sample_major" else np.ascontiguousarray(grad.transpose(1, 0, 2))
        plan = shard.plan_step(w.ids, w.offsets, w.batch)
        pooled = plan.forward()
        plan.dedup()
        plan.apply(torch.from_numpy(g).to(gpu_device))
        shard.synchronize()
        u = int(plan.unique_count.item())
        results[layout] = (_host(pooled), plan.unique[:u].cpu().numpy(), plan.inverse[:w.num_ids].cpu().numpy(),
                           plan.first_indices[:u].cpu().numpy(), _host(shard.table),
                           shard.state.state0.cpu().numpy())
    a, b = results["sample_major"], results["table_major"]
    np.testing.assert_array_equal(a[0].transpose(1, 0, 2), b[0])
    for x, y in zip(a[1:], b[1:]):
        np.testing.assert_array_equal(x, y)
    no_device_errors()


@pytest.mark.parametrize("pooling,optimizer", [("sum", "rowwise_adagrad"), ("mean", "adam"), ("weighted", "sgd"),
                                               ("sum", "none"), ("weighted", "none")])
def test_one_id_per_bag_plan_matches_oracle(gpu_device, no_device_errors, pooling, optimizer):
    """Table-major plan over bags of exactly one id: the dedup keeps no gradient row per
    occurrence (each occurrence is its own pooled row); step against the oracle."""
    from flare_amd import _native
    from flare_amd.store import Adam, PooledTableShard, RowWiseAdagrad, Sgd, Uniform
    from flare_amd.workload import make_workload, pooled_grad_host

    w = make_workload(2, batch=1800, row_scale=0.0005)
    assert np.array_equal(w.offsets, np.arange(w.offsets.size))
    weights = np.random.default_rng(4).uniform(0, 1, w.num_ids).astype(np.float32) if pooling == "weighted" else None
    opt = {"rowwise_adagrad": RowWiseAdagrad(lr=0.01, eps=1e-8), "adam": Adam(lr=0.01), "sgd": Sgd(lr=0.01),
           "none": RowWiseAdagrad()}[optimizer]
    shard = PooledTableShard(w.table_rows, w.dim, value_dtype=w.value_dtype, optimizer=opt,
                             initializer=Uniform(-0.01, 0.01), seed=9, layout="table_major")
    table0 = _host(shard.table.clone())
    grad = pooled_grad_host(w)  # [B, T, D]
    plan = shard.plan_step(w.ids, w.offsets, w.batch, pooling=pooling, per_sample_weights=weights)
    assert plan._dedup_layout & _native.LAYOUT_ONE_ID_PER_BAG
    g = torch.from_numpy(np.ascontiguousarray(grad.transpose(1, 0, 2))).to(gpu_device)
    grad_out = none_opt = None
    if optimizer == "none":
        grad_out = torch.empty((w.num_ids, w.dim), dtype=torch.float32, device=gpu_device)
        none_opt = _native.FlareOptimizer()
        none_opt.kind = _native.OPT_NONE
    pooled = plan.forward()
    plan.dedup()
    plan.apply(g, grad_out=grad_out, optimizer=none_opt)
    shard.synchronize()
    u = int(plan.unique_count.item())
    if optimizer == "none":
        eu, ei, ef, eg = O.pooled_grad_sums(w.ids, w.offsets, w.row_base(), w.batch, w.dim, grad,
                                            pooling=pooling, weights=weights)
        np.testing.assert_array_equal(plan.unique[:u].cpu().numpy(), eu)
        np.testing.assert_array_equal(plan.inverse[:w.num_ids].cpu().numpy(), ei)
        np.testing.assert_array_equal(plan.first_indices[:u].cpu().numpy(), ef)
        np.testing.assert_array_equal(grad_out[:u].cpu().numpy(), eg)
        np.testing.assert_array_equal(_host(shard.table), table0)
    else:
        state = {}
        if optimizer == "rowwise_adagrad":
            state = {"acc": np.zeros(w.total_rows, np.float32)}
        elif optimizer == "adam":
            state = {"m": np.zeros((w.total_rows, w.dim), np.float32),
                     "v": np.zeros((w.total_rows, w.dim), np.float32), "step": np.zeros(w.total_rows, np.int32)}
        e_pooled, e_table, e_state, e_unique, e_inverse, e_first = O.pooled_step(
            table0, state, w.ids, w.offsets, w.row_base(), w.batch, w.dim, grad, storage=w.value_dtype,
            pooling=pooling, weights=weights, optimizer=optimizer)
        np.testing.assert_array_equal(_host(pooled), np.ascontiguousarray(e_pooled.transpose(1, 0, 2)))
        np.testing.assert_array_equal(plan.unique[:u].cpu().numpy(), e_unique)
        np.testing.assert_array_equal(plan.inverse[:w.num_ids].cpu().numpy(), e_inverse)
        np.testing.assert_array_equal(plan.first_indices[:u].cpu().numpy(), e_first)
        ulps = O.storage_ulp_distance(_host(shard.table), e_table, w.value_dtype)
        assert ulps.max() <= 1, f"max ulp {ulps.max()}"
        if optimizer == "rowwise_adagrad":
            np.testing.assert_allclose(shard.state.state0.cpu().numpy(), e_state["acc"], rtol=1e-5, atol=0)
        elif optimizer == "adam":
            np.testing.assert_allclose(shard.state.state0.cpu().numpy(), e_state["m"], rtol=1e-5, atol=1e-12)
            np.testing.assert_array_equal(shard.state.step.cpu().numpy(), e_state["step"])
    no_device_errors()


def test_one_id_per_bag_claim_is_checked(gpu_device, no_device_errors):
    """The one-id-per-bag flag with a bag of two ids: error bit 1, no runs, no update."""
    import ctypes

    from flare_amd import _native
    from flare_amd.store import PooledTableShard, RowWiseAdagrad, Uniform

    shard = PooledTableShard([20, 20], 8, value_dtype="float32", optimizer=RowWiseAdagrad(lr=0.5),
                             initializer=Uniform(-1.0, 1.0), seed=1, layout="table_major")
    table0 = shard.table.clone()
    batch = 3
    offsets = torch.tensor([0, 1, 3, 4, 5, 6, 7], dtype=torch.int64, device=gpu_device)  # bag 1 holds 2 ids
    ids = torch.tensor([1, 2, 3, 4, 5, 6, 7], dtype=torch.int64, device=gpu_device)
    n = int(ids.numel())
    lib = _native.library()
    ws_bytes = lib.flare_pooled_backward_workspace_bytes(n, shard.total_rows, shard.dim)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=gpu_device)
    count = torch.full((1,), -1, dtype=torch.int64, device=gpu_device)
    grad = torch.ones((2, batch, 8), dtype=torch.float32, device=gpu_device)
    stream = int(torch.cuda.current_stream(gpu_device).cuda_stream)
    torch.cuda.synchronize()
    layout = _native.LAYOUT_TABLE_MAJOR | _native.LAYOUT_ONE_ID_PER_BAG
    _native.call("flare_pooled_dedup", ids.data_ptr(), _native.INT64, n, offsets.data_ptr(), 2, batch,
                 shard.row_base.data_ptr(), shard.total_rows, 8, 0, layout, None, None, count.data_ptr(),
                 ws.data_ptr(), ws_bytes, stream)
    opt = shard.state.native_optimizer
    s0, s1, st = shard.state.pointers()
    _native.call("flare_pooled_apply", shard.table.data_ptr(), _native.FLOAT32, shard.total_rows, 8, s0, s1, st,
                 ctypes.byref(opt), n, 2, batch, 0, None, grad.data_ptr(), 1, None, None, ws.data_ptr(), ws_bytes,
                 stream)
    torch.cuda.synchronize()
    assert int(count.item()) == 0
    assert torch.equal(shard.table, table0)
    no_device_errors(1)


def _one_id_forward(shard, ids, offsets, batch, pooling, weights, layout_flags):
    from flare_amd import _native
    from flare_amd.conversion import storage_code

    dev = shard.device
    d_ids = torch.from_numpy(ids).to(dev)
    d_off = torch.from_numpy(offsets).to(dev)
    d_w = None if weights is None else torch.from_numpy(weights).to(dev)
    out = torch.full((shard.num_tables, batch, shard.dim), 7.0, dtype=shard.table.dtype, device=dev)
    code = {"sum": 0, "mean": 1, "weighted": 2}[pooling]
    id_code = _native.INT32 if ids.dtype == np.int32 else _native.INT64
    _native.call("flare_gather_pooled_csr", shard.table.data_ptr(), storage_code(shard.table.dtype),
                 shard.total_rows, shard.dim, d_ids.data_ptr(), id_code, int(ids.size), d_off.data_ptr(),
                 shard.num_tables, batch, shard.row_base.data_ptr(), code, layout_flags,
                 None if d_w is None else d_w.data_ptr(), out.data_ptr(),
                 int(torch.cuda.current_stream(dev).cuda_stream))
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("pooling", ["sum", "mean", "weighted"])
@pytest.mark.parametrize("storage", ["bfloat16", "float16", "float32"])
@pytest.mark.parametrize("width", [0, 1, 2, 3, 4])
def test_one_id_forward_bit_exact(gpu_device, no_device_errors, pooling, storage, width):
    """flare_gather_pooled_csr with the one-id-per-bag flag (ids read with their offsets): rows of
    4 to 128 16-byte vectors, int32 and int64 ids, some ids past their table (error bit 1, a zero
    row); every row equals the oracle's pooling of the bag's valid ids."""
    from flare_amd import _native
    from flare_amd.store import PooledTableShard, Uniform

    dim = SHORT_DIMS[storage][width]
    rng = np.random.default_rng(31 + width)
    table_rows, batch = [9, 300, 41], 1001
    limit = np.repeat(np.asarray(table_rows), batch)
    ids = rng.integers(0, 1 << 30, size=limit.size) % limit
    bad = np.zeros(ids.size, bool)
    bad[2::53] = True
    ids = np.where(bad, limit + rng.integers(0, 4, size=ids.size), ids).astype(np.int64)
    offsets = np.arange(ids.size + 1, dtype=np.int64)
    weights = rng.uniform(0, 1, size=ids.size).astype(np.float32) if pooling == "weighted" else None
    shard = PooledTableShard(table_rows, dim, value_dtype=storage, initializer=Uniform(-1.0, 1.0), seed=width,
                             layout="table_major")
    flags = _native.LAYOUT_TABLE_MAJOR | _native.LAYOUT_ONE_ID_PER_BAG
    pooled = _one_id_forward(shard, ids.astype(np.int32) if width == 1 else ids, offsets, batch, pooling,
                             weights, flags)
    keep_off = np.zeros(ids.size + 1, np.int64)
    keep_off[1:] = np.cumsum(~bad)
    row_base = np.concatenate([[0], np.cumsum(table_rows)]).astype(np.int64)
    expected = O.gather_pooled_csr(_host(shard.table), ids[~bad], keep_off, row_base, batch, dim,
                                   storage=storage, pooling=pooling,
                                   weights=None if weights is None else weights[~bad])
    np.testing.assert_array_equal(_host(pooled), np.ascontiguousarray(expected.transpose(1, 0, 2)))
    no_device_errors(1)


def test_one_id_forward_claim_is_checked(gpu_device, no_device_errors):
    """The flag with as many ids as bags but one bag of two ids (and so one empty bag): error bit
    1, the rows of those bags are zeros, every other row is its id's row; the flag with a
    different id count is refused on the host."""
    from flare_amd import _native
    from flare_amd.store import PooledTableShard, Uniform

    shard = PooledTableShard([20, 30], 16, value_dtype="float32", initializer=Uniform(-1.0, 1.0), seed=4,
                             layout="table_major")
    batch = 4
    offsets = np.array([0, 1, 3, 3, 4, 5, 6, 7, 8], np.int64)  # bag 1 holds 2 ids, bag 2 none
    ids = np.array([1, 2, 3, 4, 5, 6, 7, 8], np.int64)
    flags = _native.LAYOUT_TABLE_MAJOR | _native.LAYOUT_ONE_ID_PER_BAG
    pooled = _one_id_forward(shard, ids, offsets, batch, "sum", None, flags).cpu().numpy().reshape(8, 16)
    table = shard.table.cpu().numpy()
    base = [0, 0, 0, 0, 20, 20, 20, 20]
    for k in range(8):
        if k in (1, 2):
            np.testing.assert_array_equal(pooled[k], np.zeros(16, np.float32))
        else:
            np.testing.assert_array_equal(pooled[k], table[base[k] + ids[k]])
    no_device_errors(1)
    with pytest.raises(ValueError):
        _one_id_forward(shard, ids[:7], offsets[:8], batch, "sum", None, flags)


# row widths for the long-bag path: 64 to 512 elements, and 96 / 32 (not multiples of 64)
LONG_DIMS = {"bfloat16": (64, 128, 256, 512, 96), "float16": (64, 128, 256, 512, 96),
             "float32": (64, 128, 256, 96, 32)}


@pytest.mark.parametrize("layout", ["sample_major", "table_major"])
@pytest.mark.parametrize("pooling", ["sum", "mean", "weighted"])
@pytest.mark.parametrize("storage", ["bfloat16", "float16", "float32"])
@pytest.mark.parametrize("width", [0, 1, 2, 3, 4])
def test_long_bag_forward_bit_exact(gpu_device, no_device_errors, layout, pooling, storage, width):
    """Bags of 8-40 ids (a few of 0, 1 and 130-300), so at least 8 per bag on average (the
    long-bag path: several rounds of prefetched ids per lane-group stream), rows of 32 to 512
    elements, int32 and int64 ids, both layouts; some ids past their table (error bit 1, pooled
    as absent); against the oracle, bit for bit."""
    from flare_amd.store import PooledTableShard, Uniform

    dim = LONG_DIMS[storage][width]
    rng = np.random.default_rng(41 + width)
    table_rows, batch = [13, 700, 90], 97
    lengths = rng.integers(8, 41, size=len(table_rows) * batch)
    lengths[3::29] = 0
    lengths[7::31] = 1
    lengths[11::50] = rng.integers(130, 301, size=lengths[11::50].size)
    offsets = np.zeros(lengths.size + 1, np.int64)
    offsets[1:] = np.cumsum(lengths)
    assert offsets[-1] >= 8 * lengths.size
    bag_table = np.repeat(np.arange(lengths.size) // batch, lengths)
    limit = np.asarray(table_rows)[bag_table]
    ids = rng.integers(0, 1 << 30, size=int(offsets[-1])) % limit
    bad = np.zeros(ids.size, bool)
    bad[5::67] = True
    ids = np.where(bad, limit + rng.integers(0, 3, size=ids.size), ids).astype(np.int64)
    weights = rng.uniform(0, 1, size=ids.size).astype(np.float32) if pooling == "weighted" else None
    shard = PooledTableShard(table_rows, dim, value_dtype=storage, initializer=Uniform(-1.0, 1.0), seed=width,
                             layout=layout)
    pooled = shard.lookup_pooled(ids.astype(np.int32) if width == 1 else ids, offsets, batch, pooling=pooling,
                                 per_sample_weights=weights)
    shard.synchronize()
    keep_len = np.add.reduceat(~bad, offsets[:-1]) * (lengths > 0)
    keep_off = np.zeros(lengths.size + 1, np.int64)
    keep_off[1:] = np.cumsum(keep_len)
    row_base = np.concatenate([[0], np.cumsum(table_rows)]).astype(np.int64)
    expected = O.gather_pooled_csr(_host(shard.table), ids[~bad], keep_off, row_base, batch, dim, storage=storage,
                                   pooling=pooling, weights=None if weights is None else weights[~bad])
    if layout == "table_major":
        expected = np.ascontiguousarray(expected.transpose(1, 0, 2))
    np.testing.assert_array_equal(_host(pooled), expected)
    no_device_errors(1)


@pytest.mark.parametrize("num_plans", [2, 3])
def test_pipeline_matches_serial_steps(gpu_device, no_device_errors, num_plans):
    """PooledStepPipeline (each batch's dedup one step ahead, on a second stream beside the
    previous update), through step() and through forward() / update(), against the same steps
    run one phase after another on another shard:
    pooled rows, dedup outputs and the final table and state bit for bit, and the
    first-step pooled rows against the oracle."""
    from flare_amd.store import PooledStepPipeline, PooledTableShard, RowWiseAdagrad, Uniform
    from flare_amd.workload import make_workload, pooled_grad_host

    ws = [make_workload(2, batch=900, row_scale=0.0005, batch_index=k) for k in range(num_plans)]
    w0 = ws[0]

    def shard():
        return PooledTableShard(w0.table_rows, w0.dim, value_dtype=w0.value_dtype,
                                optimizer=RowWiseAdagrad(lr=0.05, eps=1e-8), initializer=Uniform(-0.01, 0.01),
                                seed=21, layout="table_major")

    grads = [torch.from_numpy(np.ascontiguousarray(pooled_grad_host(w).transpose(1, 0, 2))).to(gpu_device)
             for w in ws]
    a, b = shard(), shard()
    table0 = _host(a.table.clone())
    pa = [a.plan_step(w.ids, w.offsets, w.batch) for w in ws]
    pb = [b.plan_step(w.ids, w.offsets, w.batch) for w in ws]
    pipe = PooledStepPipeline(pa)
    steps = 2 * num_plans + 1
    for i in range(steps):
        k = i % num_plans
        if i % 2:
            pooled_a = pipe.step(i, grads[k]).clone()
        else:  # the training-loop form: the gradient is given after the forward
            pooled_a = pipe.forward(i).clone()
            with pytest.raises(ValueError):
                pipe.forward(i + 1)  # the update of step i comes first
            pipe.update(i, grads[k])
        pooled_b = pb[k].forward().clone()
        pb[k].dedup()
        pb[k].apply(grads[k])
        a.synchronize()
        b.synchronize()
        np.testing.assert_array_equal(_host(pooled_a), _host(pooled_b))
        u = int(pb[k].unique_count.item())
        assert int(pa[k].unique_count.item()) == u
        np.testing.assert_array_equal(pa[k].unique[:u].cpu().numpy(), pb[k].unique[:u].cpu().numpy())
        np.testing.assert_array_equal(pa[k].inverse[:ws[k].num_ids].cpu().numpy(),
                                      pb[k].inverse[:ws[k].num_ids].cpu().numpy())
        if i == 0:
            e_pooled = O.gather_pooled_csr(table0, w0.ids, w0.offsets, w0.row_base(), w0.batch, w0.dim,
                                           storage=w0.value_dtype)
            np.testing.assert_array_equal(_host(pooled_a), np.ascontiguousarray(e_pooled.transpose(1, 0, 2)))
    pipe.finish()
    a.synchronize()
    np.testing.assert_array_equal(_host(a.table), _host(b.table))
    np.testing.assert_array_equal(a.state.state0.cpu().numpy(), b.state.state0.cpu().numpy())
    with pytest.raises(ValueError):
        pipe.step(0, grads[0])
    with pytest.raises(ValueError):
        pipe.update(steps, grads[0])  # no forward of that step
    with pytest.raises(ValueError):
        PooledStepPipeline(pa[:1])
    no_device_errors()


def test_pipeline_reduced_gradients_match_serial(gpu_device, no_device_errors):
    """The pipeline with FLARE_OPT_NONE (reduced gradients written to grad_out, the table
    untouched) over ragged weighted bags: grad_out and the dedup outputs of every step equal
    those of the same steps run one phase after another."""
    from flare_amd import _native
    from flare_amd.store import PooledStepPipeline, PooledTableShard, RowWiseAdagrad, Uniform
    from flare_amd.workload import make_workload, pooled_grad_host

    ws = [make_workload(3, batch=300, row_scale=0.0005, batch_index=k) for k in range(2)]
    w0 = ws[0]
    none_opt = _native.FlareOptimizer()
    none_opt.kind = _native.OPT_NONE

    def shard():
        return PooledTableShard(w0.table_rows, w0.dim, value_dtype=w0.value_dtype, optimizer=RowWiseAdagrad(),
                                initializer=Uniform(-0.01, 0.01), seed=4, layout="table_major")

    a, b = shard(), shard()
    table0 = _host(a.table.clone())
    pa = [a.plan_step(w.ids, w.offsets, w.batch, pooling="weighted", per_sample_weights=w.weights) for w in ws]
    pb = [b.plan_step(w.ids, w.offsets, w.batch, pooling="weighted", per_sample_weights=w.weights) for w in ws]
    grads = [torch.from_numpy(np.ascontiguousarray(pooled_grad_host(w).transpose(1, 0, 2))).to(gpu_device)
             for w in ws]
    n_max = max(w.num_ids for w in ws)
    out_a = torch.empty((n_max, w0.dim), dtype=torch.float32, device=gpu_device)
    out_b = torch.empty_like(out_a)
    pipe = PooledStepPipeline(pa)
    for i in range(5):
        k = i % 2
        pipe.step(i, grads[k], grad_out=out_a, optimizer=none_opt)
        pb[k].forward()
        pb[k].dedup()
        pb[k].apply(grads[k], grad_out=out_b, optimizer=none_opt)
        a.synchronize()
        b.synchronize()
        u = int(pb[k].unique_count.item())
        assert int(pa[k].unique_count.item()) == u
        np.testing.assert_array_equal(out_a[:u].cpu().numpy(), out_b[:u].cpu().numpy())
        np.testing.assert_array_equal(pa[k].first_indices[:u].cpu().numpy(), pb[k].first_indices[:u].cpu().numpy())
    pipe.finish()
    a.synchronize()
    np.testing.assert_array_equal(_host(a.table), table0)
    no_device_errors()
