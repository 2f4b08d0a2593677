"""Writes the golden fixtures of tests/golden (run from the repository root).

    python tests/golden/make_golden.py

Two kinds of vectors, all small:

* literal known answers from the reference's own tests (inputs and expected
  outputs copied as data, each file naming the test it comes from);
* outputs of this repository's CPU oracle (oracle/sparse_oracle.py) on
  seeded inputs, frozen so that the oracle and the HIP path are both checked
  against the same bits from one commit to the next.

The reference itself is not imported or run: its Python needs packages that
are absent here, and the literal vectors above are what its tests assert.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

from oracle import sparse_oracle as O  # noqa: E402

OUT = Path(__file__).resolve().parent

# tests/runtime/test_sparse_input_resources.py:77-123 (first-occurrence dedup)
UNIQUE_CASES = [
    (np.asarray([1, 2, 1, 3], np.int64), [1, 2, 3], [0, 1, 0, 2], [0, 1, 3]),
    (np.asarray([], np.int64), [], [], []),
    (np.asarray([7, 7, 7], np.int64), [7], [0, 0, 0], [0]),
    (np.asarray([3, 1, 3, 2, 1], np.int64), [3, 1, 2], [0, 1, 0, 2, 1], [0, 1, 3]),
    (np.asarray([-1, 0, -1, np.iinfo(np.int64).min], np.int64),
     [-1, 0, np.iinfo(np.int64).min], [0, 1, 0, 2], [0, 1, 3]),
    (np.asarray([2**63, 0, 2**63, 2**64 - 1], np.uint64), [2**63, 0, 2**64 - 1], [0, 1, 0, 2], [0, 1, 3]),
    (np.asarray([5, -2, 5, 9], np.int32), [5, -2, 9], [0, 1, 0, 2], [0, 1, 3]),
]


def unique_cases() -> None:
    arrays = {}
    for i, (values, unique, inverse, first) in enumerate(UNIQUE_CASES):
        arrays[f"case{i}_values"] = values
        arrays[f"case{i}_unique"] = np.asarray(unique, dtype=values.dtype)
        arrays[f"case{i}_inverse"] = np.asarray(inverse, np.int32)
        arrays[f"case{i}_first"] = np.asarray(first, np.int64)
    arrays["count"] = np.asarray(len(UNIQUE_CASES))
    np.savez(OUT / "unique_reference_cases.npz", **arrays)


def pooled_known_answers() -> None:
    # tests/kernels/test_sparse_embedding_backend.py:78-89 (fp32, pad row -> zeros)
    # and :162-172, :175-183 (fp16 storage with fp32 accumulation)
    np.savez(
        OUT / "gather_pooled_reference_cases.npz",
        f32_emb=np.arange(8, dtype=np.float32).reshape(4, 2),
        f32_inverse=np.asarray([0, 4, 2, 1], np.int32),
        f32_expected=np.asarray([[[0, 1]], [[0, 0]], [[4, 5]], [[2, 3]]], np.float32),
        f16_emb=np.asarray([[1.5, 2.0], [3.0, 4.0]], np.float16),
        f16_inverse=np.asarray([0, 1, 2, 2], np.int32),
        f16_expected=np.asarray([[[4.5, 6.0]], [[0.0, 0.0]]], np.float16),
        f16_wide_emb=np.asarray([[40000.0], [-40000.0], [1.0]], np.float16),
        f16_wide_inverse=np.asarray([0, 1, 2], np.int32),
        f16_wide_expected=np.asarray([[[1.0]]], np.float16),
    )


def csr_case(storage: str, pooling: str, seed: int) -> None:
    """Ragged CSR bags over 3 tables (empty bags, bags longer than an id chunk)."""
    rng = np.random.default_rng(seed)
    table_rows = np.asarray([5, 40, 17], np.int64)
    batch, dim = 7, 24
    lengths = rng.integers(0, 40, size=table_rows.size * batch)
    lengths[::5] = 0
    offsets = np.zeros(lengths.size + 1, np.int64)
    offsets[1:] = np.cumsum(lengths)
    bag_table = np.repeat(np.arange(lengths.size) // batch, lengths)
    ids = (rng.integers(0, 1 << 30, size=int(offsets[-1])) % table_rows[bag_table]).astype(np.int64)
    weights = rng.uniform(0, 1, size=ids.size).astype(np.float32) if pooling == "weighted" else None
    row_base = np.concatenate([[0], np.cumsum(table_rows)]).astype(np.int64)
    table = O.f32_to_storage(rng.uniform(-1, 1, (int(row_base[-1]), dim)).astype(np.float32), storage)
    pooled = O.gather_pooled_csr(table, ids, offsets, row_base, batch, dim, storage=storage,
                                 pooling=pooling, weights=weights)
    grad = rng.normal(0, 1, (batch, table_rows.size, dim)).astype(np.float32)
    unique, inverse, first, sums = O.pooled_grad_sums(ids, offsets, row_base, batch, dim, grad,
                                                      pooling=pooling, weights=weights)
    extra = {} if weights is None else {"weights": weights}
    np.savez(OUT / f"csr_pooled_{storage}_{pooling}.npz", table=table, ids=ids, offsets=offsets,
             row_base=row_base, batch=np.asarray(batch), dim=np.asarray(dim), pooled=pooled, grad=grad,
             unique=unique, inverse=inverse, first=first, grad_sums=sums, **extra)


def scatter_pooled_case() -> None:
    """Duplicate-key pooled scatter, checked the way the reference's tests check it:
    np.add.at over the non-pad slots in float64 (test_sparse_embedding_backend.py:353-390:
    rows=256, about 80% pad slots, tolerance 2e-4; batch 16 here instead of 48 to keep the file small)."""
    rng = np.random.default_rng(93)
    arrays = {}
    for k, (features, max_el, dim) in enumerate([(12, 30, 128), (44, 30, 40), (2, 1, 418)]):
        batch, rows = 16, 256
        inverse = rng.integers(0, rows, (batch, features, max_el)).astype(np.int32)
        inverse[rng.random(inverse.shape) < 0.8] = rows  # pad slots
        grad = rng.standard_normal((batch, features, dim)).astype(np.float32)
        expected = np.zeros((rows, dim), np.float64)
        slots = np.broadcast_to(grad[:, :, None, :], (batch, features, max_el, dim)).reshape(-1, dim)
        flat = inverse.reshape(-1)
        keep = flat != rows
        np.add.at(expected, flat[keep], slots[keep].astype(np.float64))
        arrays[f"case{k}_inverse"] = inverse
        arrays[f"case{k}_grad"] = grad
        arrays[f"case{k}_expected"] = expected.astype(np.float32)
        arrays[f"case{k}_shape"] = np.asarray([batch, features, max_el, dim, rows])
    np.savez(OUT / "scatter_pooled_seed93.npz", **arrays)


def optimizer_cases() -> None:
    # tests/runtime/test_sparse_storage_limits.py:41-119: zero-initialized rows,
    # Adam(lr=0.1), gradient of ones: -0.1 after step 1, -0.2 after step 2
    np.savez(OUT / "adam_reference_case.npz", lr=np.asarray(0.1), dim=np.asarray(4),
             keys=np.asarray([3, 7], np.int64), step1=np.full((2, 4), -0.1, np.float32),
             step2=np.full((2, 4), -0.2, np.float32))
    # tests/training/test_optimizer_factories.py:43-51 (optax adagrad, initial
    # accumulator 0.1, weight 1, gradient 2, lr 0.1): 1 - 0.1*2/sqrt(0.1 + 2^2 + 1e-8),
    # which row-wise Adagrad reproduces for a row of width 1
    w, acc = O.rowwise_adagrad_update(np.ones((1, 1), np.float32), np.full(1, 0.1, np.float32),
                                      np.full((1, 1), 2.0, np.float32), lr=0.1, eps=1e-8)
    np.savez(OUT / "adagrad_reference_case.npz", lr=np.asarray(0.1), acc0=np.asarray(0.1, np.float32),
             grad=np.asarray(2.0, np.float32), expected=np.asarray(1 - 0.1 * 2 / np.sqrt(0.1 + 4 + 1e-8)),
             oracle_w=w.reshape(()), oracle_acc=acc.reshape(()))


def pooled_step_case() -> None:
    """One full step (forward, dedup, row-wise Adagrad) on 26 small bf16 tables, bag 1, Zipf ids.

    Only the rows the step touches (the unique keys) are stored after the update.
    """
    from flare_amd.workload import make_workload

    w = make_workload(2, batch=32, row_scale=0.0001)
    rng = np.random.default_rng(21)
    table0 = O.f32_to_storage(rng.uniform(-0.01, 0.01, (w.total_rows, w.dim)).astype(np.float32), "bfloat16")
    grad = (rng.standard_normal((w.batch, w.num_tables, w.dim)) * 1e-3).astype(np.float32)
    state = {"acc": np.zeros(w.total_rows, np.float32)}
    pooled, table1, state1, unique, inverse, first = O.pooled_step(
        table0, state, w.ids, w.offsets, w.row_base(), w.batch, w.dim, grad, storage="bfloat16",
        optimizer="rowwise_adagrad")
    np.savez_compressed(OUT / "pooled_step_26x128_bf16.npz", table0=table0, ids=w.ids, offsets=w.offsets,
                        row_base=w.row_base(), table_rows=np.asarray(w.table_rows, np.int64),
                        batch=np.asarray(w.batch), dim=np.asarray(w.dim), grad=grad, pooled=pooled,
                        rows1=table1[unique], acc1=state1["acc"][unique], unique=unique, inverse=inverse,
                        first=first)


def main() -> None:
    unique_cases()
    pooled_known_answers()
    seed = 300
    for storage in ("float32", "float16", "bfloat16"):
        for pooling in ("sum", "mean", "weighted"):
            csr_case(storage, pooling, seed)
            seed += 1
    scatter_pooled_case()
    optimizer_cases()
    pooled_step_case()
    for f in sorted(OUT.glob("*.npz")):
        print(f"{f.name:40s} {f.stat().st_size:8d} bytes")


if __name__ == "__main__":
    main()
