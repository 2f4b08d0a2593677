"""Pins the C restatement (CPU baseline) against the numpy oracle (CPU only)."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import cpu_step as C
from oracle import sparse_oracle as O


def test_fp16_conversions_match_numpy():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(20000).astype(np.float32) * np.float32(100),
                        rng.standard_normal(2000).astype(np.float32) * np.float32(1e-6),
                        np.asarray([0, -0.0, 65504, 65519.9, 65520, -70000, 6e-8, 3e-8, 2.9e-8, np.inf, -np.inf], np.float32)])
    table = x.reshape(-1, 1)
    # round trip through the C storage path: forward of a single-id bag copies x -> fp16
    ids = np.arange(x.size)
    offsets = np.arange(x.size + 1)
    with np.errstate(over="ignore"):
        out = C.pooled_forward(table.astype(np.float16), "float16", 1, ids, offsets, 1, x.size, np.asarray([0, x.size]))
        np.testing.assert_array_equal(out.reshape(-1), x.astype(np.float16))
    bits = C.pooled_forward(O.f32_to_bf16_bits(x).reshape(-1, 1), "bfloat16", 1, ids, offsets, 1, x.size,
                            np.asarray([0, x.size]))
    # pooling adds onto +0.0, so -0.0 comes back as +0.0 (as in the reference): compare values
    np.testing.assert_array_equal(O.bf16_bits_to_f32(bits.reshape(-1)), O.bf16_bits_to_f32(O.f32_to_bf16_bits(x)))


@pytest.mark.parametrize("config,storage", [(1, "float32"), (2, "bfloat16"), (3, "float16")])
@pytest.mark.parametrize("pooling", ["sum", "mean", "weighted"])
def test_forward_matches_oracle_bitwise(config, storage, pooling):
    from flare_amd.workload import make_workload

    w = make_workload(config, batch=200, row_scale=0.0005)
    table = C.init_table(w.total_rows, w.dim, storage, -0.05, 0.05, 7)
    weights = w.weights if w.weights is not None else np.random.default_rng(1).random(w.num_ids, dtype=np.float32)
    got = C.pooled_forward(table, storage, w.dim, w.ids, w.offsets, w.num_tables, w.batch, w.row_base(),
                           pooling, weights)
    exp = O.gather_pooled_csr(table, w.ids, w.offsets, w.row_base(), w.batch, w.dim, storage=storage,
                              pooling=pooling, weights=weights)
    np.testing.assert_array_equal(got, exp)


@pytest.mark.parametrize("optimizer", ["rowwise_adagrad", "adam", "sgd"])
def test_backward_matches_oracle(optimizer):
    from flare_amd.workload import make_workload, pooled_grad_host

    w = make_workload(4, batch=256, row_scale=0.0002)
    storage = "bfloat16"
    table = C.init_table(w.total_rows, w.dim, storage, -0.01, 0.01, 3)
    grad = pooled_grad_host(w)
    if optimizer == "adam":
        state = {"m": np.zeros((w.total_rows, w.dim), np.float32), "v": np.zeros((w.total_rows, w.dim), np.float32),
                 "step": np.zeros(w.total_rows, np.int32)}
    elif optimizer == "rowwise_adagrad":
        state = {"acc": np.zeros(w.total_rows, np.float32)}
    else:
        state = {}
    e_pooled, e_table, e_state, eu, ei, ef = O.pooled_step(
        table, state, w.ids, w.offsets, w.row_base(), w.batch, w.dim, grad, storage=storage, optimizer=optimizer)
    t = table.copy()
    s = {k: v.copy() for k, v in state.items()}
    u, unique, inverse, _ = C.pooled_backward(t, storage, w.dim, s, optimizer, w.ids, w.offsets, w.num_tables,
                                              w.batch, w.row_base(), grad)
    assert u == eu.size
    # per-table dedup: local unique ids and local inverse, tables concatenated
    lengths = np.diff(w.offsets)
    bag = np.repeat(np.arange(w.num_tables * w.batch), lengths)
    table_of = bag // w.batch
    for tt in range(w.num_tables):
        sel = table_of == tt
        lu, li, _ = O.unique_first_occurrence_hash(w.ids[sel])
        lo = w.offsets[tt * w.batch]
        np.testing.assert_array_equal(unique[lo:lo + lu.size], lu)
        np.testing.assert_array_equal(inverse[lo:lo + li.size], li)
    # values: the C path sums in slot order, the oracle in unit order -> within 1 ulp,
    # except where a key's gradients cancel (|sum| tiny) and Adam's g/(|g|+eps)
    # amplifies the order-dependent rounding of the sum
    ulps = O.storage_ulp_distance(t, e_table, storage)
    bad = ulps > 1
    if optimizer == "adam" and bad.any():
        keys, _, _, sums = O.pooled_grad_sums(w.ids, w.offsets, w.row_base(), w.batch, w.dim, grad)
        gfull = np.zeros((w.total_rows, w.dim), np.float32)
        gfull[keys] = sums
        assert np.all(np.abs(gfull[bad]) < 1e-6), "large ulp error outside cancellation"
    else:
        assert ulps.max() <= 1
    # Two summation orders of n terms differ by at most 2 (n - 1) eps32 sum|g_i|
    # per key and element; m inherits (1 - beta1) of that, v and acc are relative.
    keys, _, _, abs_sums = O.pooled_grad_sums(w.ids, w.offsets, w.row_base(), w.batch, w.dim, np.abs(grad))
    counts = np.bincount(w.global_keys(), minlength=w.total_rows)
    bound = np.zeros((w.total_rows, w.dim), np.float64)
    bound[keys] = 2.0 * np.maximum(counts[keys] - 1, 0)[:, None] * 2.0**-24 * abs_sums
    for k in s:
        if k == "step":
            np.testing.assert_array_equal(s[k], e_state[k])
        elif k == "m":
            assert np.all(np.abs(s[k] - e_state[k]) <= 0.1 * bound * 1.01 + 1e-5 * np.abs(e_state[k]))
        elif k == "v":  # v = (1 - beta2) g^2: |dv| <= 0.001 (2|g| + dg) dg
            _, _, _, sums = O.pooled_grad_sums(w.ids, w.offsets, w.row_base(), w.batch, w.dim, grad)
            g = np.zeros((w.total_rows, w.dim), np.float64)
            g[keys] = np.abs(sums)
            assert np.all(np.abs(s[k] - e_state[k]) <= 0.001 * (2 * g + bound) * bound * 1.01 + 1e-5 * np.abs(e_state[k]))
        else:
            np.testing.assert_allclose(s[k], e_state[k], rtol=1e-4, atol=1e-15)
