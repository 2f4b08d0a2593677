"""The HIP path against the committed golden fixtures, through the C-ABI.

Same fixtures as tests/test_golden.py (literal known answers of the
reference's tests and frozen oracle outputs): indices bit-exact, pooled rows
and reduced gradients bit-exact (same fp32 order), updated rows within 1 ulp
of the storage dtype, optimizer state within rtol 1e-5, the pooled scatter
within the reference's own 2e-4 of np.add.at.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import sparse_oracle as O

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"


def load(name: str):
    return np.load(GOLDEN / name, allow_pickle=False)


def _host(t) -> np.ndarray:
    """Host copy of a torch tensor or of the operator's DeviceArray (bf16 as raw bits)."""
    from flare_amd.array import DeviceArray

    if isinstance(t, DeviceArray):
        t = t.tensor
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).cpu().numpy().view(np.uint16)
    return t.cpu().numpy()


def _set_table(shard, table: np.ndarray) -> None:
    if shard.table.dtype == torch.bfloat16:
        src = torch.from_numpy(np.ascontiguousarray(table).view(np.int16)).view(torch.bfloat16)
    else:
        src = torch.from_numpy(np.ascontiguousarray(table))
    with torch.cuda.stream(shard.stream):
        shard.table.copy_(src.to(shard.device))


def test_unique_reference_cases(gpu_device, no_device_errors):
    from flare_amd.unique import unique_first_occurrence

    f = load("unique_reference_cases.npz")
    for i in range(int(f["count"])):
        u, inv, first = unique_first_occurrence(f[f"case{i}_values"])
        np.testing.assert_array_equal(u, f[f"case{i}_unique"])
        np.testing.assert_array_equal(inv, f[f"case{i}_inverse"])
        np.testing.assert_array_equal(first, f[f"case{i}_first"])
    no_device_errors()


def test_gather_pooled_reference_cases(gpu_device, no_device_errors):
    from flare_amd.operator import HipSparseEmbeddingOperator

    f = load("gather_pooled_reference_cases.npz")
    op = HipSparseEmbeddingOperator("float32", "float32", empty_cache=False)
    out = op.gather_pooled(torch.from_numpy(f["f32_emb"]).to(gpu_device), f["f32_inverse"], 4, 2, (1, 1), 4)
    op.stream.synchronize()
    np.testing.assert_array_equal(_host(out), f["f32_expected"])
    op = HipSparseEmbeddingOperator("float16", "float32", empty_cache=False)
    for emb, inv, exp, batch, dim, widths, pad in (("f16_emb", "f16_inverse", "f16_expected", 2, 2, (1, 2), 2),
                                                   ("f16_wide_emb", "f16_wide_inverse", "f16_wide_expected",
                                                    1, 1, (1, 3), 3)):
        out = op.gather_pooled(torch.from_numpy(f[emb]).to(gpu_device), f[inv], batch, dim, widths, pad)
        op.stream.synchronize()
        np.testing.assert_array_equal(_host(out), f[exp])
    no_device_errors()


@pytest.mark.parametrize("storage", ["float32", "float16", "bfloat16"])
@pytest.mark.parametrize("pooling", ["sum", "mean", "weighted"])
def test_csr_fixtures(gpu_device, no_device_errors, storage, pooling):
    from flare_amd.store import PooledTableShard

    f = load(f"csr_pooled_{storage}_{pooling}.npz")
    w = f["weights"] if pooling == "weighted" else None
    rb = f["row_base"]
    shard = PooledTableShard(np.diff(rb).tolist(), int(f["dim"]), value_dtype=storage)
    _set_table(shard, f["table"])
    batch = int(f["batch"])
    pooled = shard.lookup_pooled(f["ids"], f["offsets"], batch, pooling=pooling, per_sample_weights=w)
    u, inv, first, g = shard.reduce_pooled_gradients(f["ids"], f["offsets"], batch, f["grad"], pooling=pooling,
                                                     per_sample_weights=w)
    shard.synchronize()
    np.testing.assert_array_equal(_host(pooled), f["pooled"])
    np.testing.assert_array_equal(u.cpu().numpy(), f["unique"])
    np.testing.assert_array_equal(inv.cpu().numpy(), f["inverse"])
    np.testing.assert_array_equal(first.cpu().numpy(), f["first"])
    np.testing.assert_array_equal(g.cpu().numpy(), f["grad_sums"])
    no_device_errors()


def test_scatter_pooled_matches_add_at(gpu_device, no_device_errors):
    from flare_amd.operator import HipSparseEmbeddingOperator

    f = load("scatter_pooled_seed93.npz")
    op = HipSparseEmbeddingOperator("float32", "float32", empty_cache=False)
    for k in range(3):
        batch, features, max_el, dim, rows = (int(x) for x in f[f"case{k}_shape"])
        inverse = torch.from_numpy(f[f"case{k}_inverse"].reshape(-1)).to(gpu_device)
        grad = torch.from_numpy(f[f"case{k}_grad"]).to(gpu_device)
        got = op.scatter_pooled(rows, dim, inverse, rows, grad, (features, max_el))
        op.stream.synchronize()
        np.testing.assert_allclose(_host(got), f[f"case{k}_expected"], rtol=2e-4, atol=2e-4)
    no_device_errors()


def test_adam_reference_case(gpu_device, no_device_errors):
    from flare_amd.store import Adam, EmbeddingStore, Zeros

    f = load("adam_reference_case.npz")
    dim = int(f["dim"])
    keys = f["keys"]
    store = EmbeddingStore(capacity=16, dims=[dim], value_dtype="float32", optimizer=Adam(lr=float(f["lr"])),
                           initializer=Zeros())
    store.lookup_or_insert(keys, dim)
    for expected in (f["step1"], f["step2"]):
        store.accumulate_gradients(keys, np.ones((keys.size, dim), np.float32))
        store.optimizer_step(1)
        values, _ = store.lookup(keys, dim)
        store.synchronize()
        np.testing.assert_allclose(values.cpu().numpy(), expected, rtol=1e-5, atol=1e-6)
    no_device_errors()


def test_adagrad_reference_case(gpu_device, no_device_errors):
    from flare_amd.store import PooledTableShard, RowWiseAdagrad

    f = load("adagrad_reference_case.npz")
    shard = PooledTableShard([1], 1, value_dtype="float32", optimizer=RowWiseAdagrad(lr=float(f["lr"]), eps=1e-8))
    _set_table(shard, np.ones((1, 1), np.float32))
    with torch.cuda.stream(shard.stream):
        shard.state.state0.fill_(float(f["acc0"]))
    shard.apply_pooled_gradients(np.zeros(1, np.int64), np.asarray([0, 1], np.int64), 1,
                                 np.full((1, 1, 1), f["grad"], np.float32))
    shard.synchronize()
    got = shard.table.cpu().numpy().reshape(())
    np.testing.assert_allclose(got, f["expected"], rtol=1e-6)
    assert got == f["oracle_w"]
    assert shard.state.state0.cpu().numpy().reshape(()) == f["oracle_acc"]
    no_device_errors()


def test_pooled_step_fixture(gpu_device, no_device_errors):
    from flare_amd.store import PooledTableShard, RowWiseAdagrad

    f = load("pooled_step_26x128_bf16.npz")
    shard = PooledTableShard(f["table_rows"].tolist(), int(f["dim"]), value_dtype="bfloat16",
                             optimizer=RowWiseAdagrad(lr=0.01, eps=1e-8))
    _set_table(shard, f["table0"])
    batch = int(f["batch"])
    pooled = shard.lookup_pooled(f["ids"], f["offsets"], batch)
    u, inv, first = shard.apply_pooled_gradients(f["ids"], f["offsets"], batch, f["grad"], return_dedup=True)
    shard.synchronize()
    np.testing.assert_array_equal(_host(pooled), f["pooled"])
    np.testing.assert_array_equal(u.cpu().numpy(), f["unique"])
    np.testing.assert_array_equal(inv.cpu().numpy(), f["inverse"])
    np.testing.assert_array_equal(first.cpu().numpy(), f["first"])
    table = _host(shard.table)
    keys = f["unique"]
    assert O.storage_ulp_distance(table[keys], f["rows1"], "bfloat16").max() <= 1
    np.testing.assert_allclose(shard.state.state0.cpu().numpy()[keys], f["acc1"], rtol=1e-5, atol=0)
    untouched = np.ones(table.shape[0], bool)
    untouched[keys] = False
    np.testing.assert_array_equal(table[untouched], f["table0"][untouched])
    no_device_errors()
