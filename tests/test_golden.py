"""The oracle against the committed golden fixtures (CPU only).

The fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py) hold
the literal known answers of the reference's tests and frozen oracle outputs;
here every one is recomputed with the oracle and compared bit for bit (the
literal float answers within the tolerance the reference's test states).
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from oracle import sparse_oracle as O

GOLDEN = Path(__file__).resolve().parent / "golden"


def load(name: str):
    return np.load(GOLDEN / name, allow_pickle=False)


def test_unique_reference_cases():
    f = load("unique_reference_cases.npz")
    for i in range(int(f["count"])):
        values = f[f"case{i}_values"]
        for fn in (O.unique_first_occurrence_hash, O.unique_first_occurrence_sorted):
            u, inv, first = fn(values)
            np.testing.assert_array_equal(u, f[f"case{i}_unique"])
            np.testing.assert_array_equal(inv, f[f"case{i}_inverse"])
            np.testing.assert_array_equal(first, f[f"case{i}_first"])


def test_gather_pooled_reference_cases():
    f = load("gather_pooled_reference_cases.npz")
    out = O.gather_pooled(f["f32_emb"], f["f32_inverse"], 4, 2, (1, 1), 4)
    np.testing.assert_array_equal(out, f["f32_expected"])
    out = O.gather_pooled(f["f16_emb"], f["f16_inverse"], 2, 2, (1, 2), 2, storage="float16")
    np.testing.assert_array_equal(out, f["f16_expected"])
    out = O.gather_pooled(f["f16_wide_emb"], f["f16_wide_inverse"], 1, 1, (1, 3), 3, storage="float16")
    np.testing.assert_array_equal(out, f["f16_wide_expected"])


@pytest.mark.parametrize("storage", ["float32", "float16", "bfloat16"])
@pytest.mark.parametrize("pooling", ["sum", "mean", "weighted"])
def test_csr_fixtures_reproduce(storage, pooling):
    f = load(f"csr_pooled_{storage}_{pooling}.npz")
    w = f["weights"] if pooling == "weighted" else None
    batch, dim = int(f["batch"]), int(f["dim"])
    pooled = O.gather_pooled_csr(f["table"], f["ids"], f["offsets"], f["row_base"], batch, dim,
                                 storage=storage, pooling=pooling, weights=w)
    np.testing.assert_array_equal(pooled, f["pooled"])
    u, inv, first, sums = O.pooled_grad_sums(f["ids"], f["offsets"], f["row_base"], batch, dim, f["grad"],
                                             pooling=pooling, weights=w)
    for got, key in ((u, "unique"), (inv, "inverse"), (first, "first"), (sums, "grad_sums")):
        np.testing.assert_array_equal(got, f[key])


def test_scatter_pooled_matches_add_at():
    # the reference checks its pooled scatter against np.add.at within 2e-4
    f = load("scatter_pooled_seed93.npz")
    for k in range(3):
        batch, features, max_el, dim, rows = (int(x) for x in f[f"case{k}_shape"])
        got = O.scatter_pooled(rows, dim, f[f"case{k}_inverse"].reshape(-1), rows, f[f"case{k}_grad"],
                               (features, max_el))
        np.testing.assert_allclose(got, f[f"case{k}_expected"], rtol=2e-4, atol=2e-4)


def test_adam_reference_case():
    f = load("adam_reference_case.npz")
    dim = int(f["dim"])
    w = np.zeros((2, dim), np.float32)
    m = np.zeros_like(w)
    v = np.zeros_like(w)
    step = np.zeros(2, np.int32)
    g = np.ones_like(w)
    for expected in (f["step1"], f["step2"]):
        w, m, v, step = O.adam_update(w, m, v, step, g, lr=float(f["lr"]))
        np.testing.assert_allclose(w, expected, rtol=1e-5, atol=1e-6)


def test_adagrad_reference_case():
    f = load("adagrad_reference_case.npz")
    w, acc = O.rowwise_adagrad_update(np.ones((1, 1), np.float32), np.full(1, f["acc0"], np.float32),
                                      np.full((1, 1), f["grad"], np.float32), lr=float(f["lr"]), eps=1e-8)
    np.testing.assert_allclose(w.reshape(()), f["expected"], rtol=1e-6)
    assert w.reshape(()) == f["oracle_w"] and acc.reshape(()) == f["oracle_acc"]


def test_pooled_step_fixture_reproduces():
    f = load("pooled_step_26x128_bf16.npz")
    batch, dim = int(f["batch"]), int(f["dim"])
    state = {"acc": np.zeros(f["table0"].shape[0], np.float32)}
    pooled, table1, state1, u, inv, first = O.pooled_step(
        f["table0"], state, f["ids"], f["offsets"], f["row_base"], batch, dim, f["grad"],
        storage="bfloat16", optimizer="rowwise_adagrad")
    np.testing.assert_array_equal(pooled, f["pooled"])
    np.testing.assert_array_equal(u, f["unique"])
    np.testing.assert_array_equal(inv, f["inverse"])
    np.testing.assert_array_equal(first, f["first"])
    np.testing.assert_array_equal(table1[u], f["rows1"])
    np.testing.assert_array_equal(state1["acc"][u], f["acc1"])
    untouched = np.ones(table1.shape[0], bool)
    untouched[u] = False
    np.testing.assert_array_equal(table1[untouched], f["table0"][untouched])
