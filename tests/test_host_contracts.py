"""Host-side contracts of the drop-in boundary (CPU only).

Follows the reference's contract tests: dtype whitelists and messages
(src/flare/runtime/sparse_precision.py:20-49,
tests/kernels/test_sparse_embedding_backend.py:130-141), target widths
(src/flare/ops/contracts.py:7-19), factory errors (src/flare/ops/factory.py:45-48),
pool-reclaimer policies (tests/kernels/test_cupy_memory.py:35-70), and the
synthetic workload generators.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import flare_amd
from flare_amd import precision
from flare_amd.contracts import pooled_sparse_widths


def test_pooled_widths_contract():
    assert pooled_sparse_widths((3, 7)) == (3, 7)
    with pytest.raises(ValueError, match="exactly two target widths"):
        pooled_sparse_widths((1, 2, 3))
    with pytest.raises(ValueError, match="positive target widths"):
        pooled_sparse_widths((0, 2))


def test_value_and_gradient_dtype_whitelists():
    assert precision.require_sparse_value_dtype("float16") == "float16"
    assert precision.require_sparse_value_dtype("bfloat16") == "bfloat16"  # documented extension
    with pytest.raises(ValueError, match="float32"):
        precision.require_sparse_gradient_dtype("float16")
    with pytest.raises(ValueError, match="must be one of"):
        precision.require_sparse_value_dtype("float64")
    with pytest.raises(ValueError):
        precision.require_sparse_optimizer_dtype("bfloat16")


def test_operator_requires_explicit_gradient_dtype():
    from flare_amd.operator import HipSparseEmbeddingOperator

    with pytest.raises(TypeError):
        HipSparseEmbeddingOperator(value_dtype="float16")  # type: ignore[call-arg]
    with pytest.raises(ValueError, match="float32"):
        HipSparseEmbeddingOperator(value_dtype="float16", gradient_dtype="float16")


def test_factory_rejects_unknown_backend():
    with pytest.raises(ValueError, match="Unknown sparse embedding operator backend 'cupy'"):
        flare_amd.create_sparse_embedding_operator("cupy", value_dtype="float16", gradient_dtype="float32")


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-GPU failure mode")
def test_operator_fails_loudly_without_gpu():
    with pytest.raises(RuntimeError, match="requires a ROCm GPU"):
        flare_amd.create_sparse_embedding_operator("hip", value_dtype="float16", gradient_dtype="float32")


def test_reclaimer_policies():
    from flare_amd.operator import EagerPoolReclaimer, RetainPoolReclaimer

    calls = []

    class _Cuda:
        @staticmethod
        def empty_cache():
            calls.append("empty")

    class _Torch:
        cuda = _Cuda

    EagerPoolReclaimer().after_operation(_Torch)
    RetainPoolReclaimer().after_operation(_Torch)
    assert calls == ["empty"]


def test_execution_context_runs_reclaimer_last():
    from flare_amd.operator import HipSparseEmbeddingOperator

    events = []

    class _Stream:
        def __enter__(self):
            events.append("enter")
            return self

        def __exit__(self, *exc):
            events.append("exit")

    class _Policy:
        def after_operation(self, _torch):
            events.append("reclaim")

    op = object.__new__(HipSparseEmbeddingOperator)
    op.stream = _Stream()
    op._memory_reclaimer = _Policy()
    with op.execution_context():
        events.append("work")
    assert events == ["enter", "work", "reclaim", "exit"]


def test_native_gradient_cast_contract():
    g = torch.ones(3, 2, dtype=torch.bfloat16)
    out = precision.prepare_sparse_native_gradient(g, transport_dtype="bfloat16", native_dtype="float32")
    assert out.dtype == torch.float32
    with pytest.raises(TypeError, match="transport dtype mismatch"):
        precision.prepare_sparse_native_gradient(g, transport_dtype="float32", native_dtype="float32")
    with pytest.raises(FloatingPointError):
        precision.prepare_sparse_native_gradient(torch.tensor([float("nan")]), transport_dtype="float32",
                                                 native_dtype="float32", validate_values=True)


def test_optimizer_config_mapping():
    from dataclasses import dataclass

    from flare_amd.store import Adam, Sgd, optimizer_from_config

    @dataclass(frozen=True)
    class SparseOptimizerConfig:  # sparse_table/contracts.py:14-25 defaults
        kind: str = "adam"
        learning_rate: float = 0.01
        beta1: float = 0.9
        beta2: float = 0.999
        eps: float = 1e-8
        weight_decay: float = 0.0
        dynamic_lr_policy: str = "constant"

    assert optimizer_from_config(SparseOptimizerConfig()) == Adam(0.01, 0.9, 0.999, 1e-8, 0.0, "constant")
    assert isinstance(optimizer_from_config(SparseOptimizerConfig(kind="sgd")), Sgd)
    with pytest.raises(ValueError, match="unsupported sparse optimizer"):
        optimizer_from_config(SparseOptimizerConfig(kind="lamb"))


@pytest.mark.parametrize("config", [1, 2, 3, 4, 5])
def test_workloads_are_seeded_and_well_formed(config):
    from flare_amd.workload import make_workload

    a = make_workload(config, batch=128, row_scale=0.001)
    b = make_workload(config, batch=128, row_scale=0.001)
    np.testing.assert_array_equal(a.ids, b.ids)
    assert a.offsets[0] == 0 and a.offsets[-1] == a.ids.size and np.all(np.diff(a.offsets) >= 0)
    assert a.offsets.size == a.num_tables * a.batch + 1
    lengths = np.diff(a.offsets)
    tables = np.repeat(np.arange(a.num_tables * a.batch), lengths) // a.batch
    assert np.all(a.ids >= 0) and np.all(a.ids < np.asarray(a.table_rows)[tables])
    c = make_workload(config, batch=128, row_scale=0.001, batch_index=1)
    assert not np.array_equal(a.ids, c.ids)


def test_zipf_head_frequency_matches_closed_form():
    from flare_amd.workload import bounded_zipf

    rng = np.random.default_rng(0)
    rows, alpha = 1000, 1.1
    ranks = bounded_zipf(rng, 400000, rows, alpha)
    p = (np.arange(1, rows + 1) ** -alpha)
    p /= p.sum()
    freq = np.bincount(ranks, minlength=rows) / ranks.size
    np.testing.assert_allclose(freq[:5], p[:5], rtol=0.03)
    assert ranks.min() >= 0 and ranks.max() < rows
