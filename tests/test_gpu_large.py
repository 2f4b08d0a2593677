"""A table of 17M rows x 128 bf16: row * dim passes 2^31 and ids sit above row 2^24.

The fused step (forward, dedup, row-wise Adagrad update) is compared with the oracle on every
touched row.  The oracle works on a compact copy of the touched rows: their keys keep their
order, so the sort, the reduction units and the dedup are the same.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import sparse_oracle as O

pytestmark = pytest.mark.gpu


def _bits(t: torch.Tensor) -> np.ndarray:
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).cpu().numpy().view(np.uint16)
    return t.cpu().numpy()


@pytest.mark.parametrize("layout", ["table_major", "sample_major"])
def test_step_on_a_table_past_2_to_the_31_elements(gpu_device, no_device_errors, layout):
    from flare_amd.store import PooledTableShard, RowWiseAdagrad, Uniform

    table_rows = [1000, 17_000_000]
    dim, batch = 128, 4096
    assert (table_rows[1] - 1) * dim > 2 ** 31
    rng = np.random.default_rng(2024)
    lengths = rng.integers(1, 4, size=2 * batch)
    offsets = np.zeros(lengths.size + 1, np.int64)
    offsets[1:] = np.cumsum(lengths)
    n0 = int(offsets[batch])
    n1 = int(offsets[-1]) - n0
    ids0 = rng.integers(0, table_rows[0], size=n0)
    hot = rng.integers(table_rows[1] - 3000, table_rows[1], size=n1)   # above row 2^24, duplicated
    ids1 = np.where(rng.random(n1) < 0.3, rng.integers(0, table_rows[1], size=n1), hot)
    ids = np.concatenate([ids0, ids1]).astype(np.int64)
    shard = PooledTableShard(table_rows, dim, value_dtype="bfloat16", optimizer=RowWiseAdagrad(lr=0.01, eps=1e-8),
                             initializer=Uniform(-0.01, 0.01), seed=6, layout=layout)
    row_base = np.asarray([0, table_rows[0], sum(table_rows)], np.int64)
    bag_of = np.repeat(np.arange(2 * batch), lengths)
    keys = row_base[bag_of // batch] + ids
    assert keys.max() >= 2 ** 24
    touched = np.unique(keys)
    idx = torch.from_numpy(touched).to(gpu_device)
    before = _bits(shard.table.index_select(0, idx))
    untouched = np.setdiff1d(rng.integers(0, row_base[-1], size=4096), touched)
    still_before = _bits(shard.table.index_select(0, torch.from_numpy(untouched).to(gpu_device)))
    grad_bm = rng.normal(0, 1e-3, size=(batch, 2, dim)).astype(np.float32)
    grad = grad_bm if layout == "sample_major" else np.ascontiguousarray(grad_bm.transpose(1, 0, 2))
    pooled = shard.lookup_pooled(ids, offsets, batch)
    unique, inverse, first = shard.apply_pooled_gradients(ids, offsets, batch, grad, return_dedup=True)
    shard.synchronize()
    after = _bits(shard.table.index_select(0, idx))
    acc_after = shard.state.state0.index_select(0, idx).cpu().numpy()
    still_after = _bits(shard.table.index_select(0, torch.from_numpy(untouched).to(gpu_device)))
    # the oracle on the compact rows: bags in table-major order as one table of 2*batch bags
    compact_ids = np.searchsorted(touched, keys)
    e_pooled, e_table, e_state, e_unique, e_inverse, e_first = O.pooled_step(
        before, {"acc": np.zeros(touched.size, np.float32)}, compact_ids, offsets,
        np.asarray([0, touched.size], np.int64), 2 * batch, dim,
        grad_bm.transpose(1, 0, 2).reshape(2 * batch, 1, dim), storage="bfloat16")
    got_pooled = _bits(pooled)
    if layout == "sample_major":
        got_pooled = got_pooled.transpose(1, 0, 2)
    np.testing.assert_array_equal(got_pooled.reshape(-1, dim), e_pooled.reshape(-1, dim))
    np.testing.assert_array_equal(unique.cpu().numpy(), touched[e_unique])
    np.testing.assert_array_equal(inverse.cpu().numpy(), e_inverse)
    np.testing.assert_array_equal(first.cpu().numpy(), e_first)
    assert O.storage_ulp_distance(after, e_table, "bfloat16").max() <= 1
    np.testing.assert_allclose(acc_after, e_state["acc"], rtol=1e-5, atol=0)
    np.testing.assert_array_equal(still_after, still_before)
    no_device_errors()
