"""Operator contract of the sparse path.

``SparseEmbeddingOperator`` keeps the method set and signatures of
``src/flare/kernels/contracts.py:16-104``; ``pooled_sparse_widths`` and the
backend list follow ``src/flare/ops/contracts.py:4-19``.  The reference's
constructor takes a Fluxway ``TensorBackend``; here the backend is torch on
the operator's device, so the constructor takes the dtypes only.
"""

from __future__ import annotations

from abc import ABC, abstractmethod
from contextlib import AbstractContextManager
from typing import Any

import numpy as np

from flare_amd.precision import require_sparse_gradient_dtype, require_sparse_value_dtype

SparsePooledWidths = tuple[int, ...]
# The reference's names ("cupy", "cpu_numba", "jax") plus this library's "hip".
SPARSE_EMBEDDING_OPERATOR_BACKENDS = ("hip",)


def pooled_sparse_widths(target_widths: SparsePooledWidths) -> tuple[int, int]:
    """Exactly two positive widths ``(F, M)`` (``src/flare/ops/contracts.py:7-19``)."""
    if len(target_widths) != 2:
        raise ValueError(
            "Sparse embedding pooled operations require exactly two target widths, "
            f"got {target_widths}."
        )
    feature_count, max_elements = (int(value) for value in target_widths)
    if feature_count <= 0 or max_elements <= 0:
        raise ValueError(
            "Sparse embedding pooled operations require positive target widths, "
            f"got {target_widths}."
        )
    return feature_count, max_elements


class SparseEmbeddingOperator(ABC):
    inverse_host_dtype = np.int32

    def __init__(self, value_dtype: str, gradient_dtype: str):
        self.value_dtype = require_sparse_value_dtype(value_dtype)
        self.gradient_dtype = require_sparse_gradient_dtype(gradient_dtype)

    def to_dlpack(self, value: Any) -> Any:
        if hasattr(value, "__dlpack__"):
            return value.__dlpack__()
        raise TypeError(
            f"Value of type {type(value).__name__} does not support DLPack protocol."
        )

    def local_array(self, value: Any) -> Any:
        # First addressable shard of a distributed array (conversion.py:130-141).
        if hasattr(value, "addressable_shards"):
            shards = value.addressable_shards
            if not shards:
                raise ValueError("No addressable shards found in distributed array.")
            value = shards[0].data
        return self.array(value)

    @abstractmethod
    def array(self, value: Any) -> Any:
        raise NotImplementedError

    @abstractmethod
    def inverse(self, value: Any) -> Any:
        raise NotImplementedError

    @abstractmethod
    def gather(self, emb_flat: Any, inverse: Any, batch_size: int, emb_dim: int,
               pad_index: int) -> Any:
        raise NotImplementedError

    @abstractmethod
    def gather_pooled(self, emb_flat: Any, inverse: Any, batch_size: int, emb_dim: int,
                      target_widths: tuple[int, ...], pad_index: int) -> Any:
        raise NotImplementedError

    @abstractmethod
    def scatter(self, emb_rows: int, emb_dim: int, inverse: Any, pad_index: int,
                gradient: Any) -> Any:
        raise NotImplementedError

    @abstractmethod
    def scatter_pooled(self, emb_rows: int, emb_dim: int, inverse: Any, pad_index: int,
                       gradient: Any, target_widths: tuple[int, ...]) -> Any:
        raise NotImplementedError

    @abstractmethod
    def execution_context(self) -> AbstractContextManager[Any]:
        raise NotImplementedError

    @abstractmethod
    def prewarm(self) -> None:
        raise NotImplementedError
