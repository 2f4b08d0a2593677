"""MI355X (gfx950) sparse-embedding hot path of Flare, as hand-written HIP.

Public surface (mirrors the reference's operator, dedup and store interfaces):

* ``create_sparse_embedding_operator("hip", value_dtype=..., gradient_dtype=...)``
  -> ``HipSparseEmbeddingOperator`` (``gather``, ``gather_pooled``, ``scatter``,
  ``scatter_pooled``, ``execution_context``, ``prewarm``)
* ``unique_first_occurrence(values)``
* ``EmbeddingStore`` (lookup / accumulate_gradients / optimizer_step)
* ``PooledTableShard`` (fused CSR pooled lookup and pooled-gradient update)

Importing the package does not touch the GPU; the HIP library is loaded on
first use and its absence raises ``RuntimeError`` (there is no CPU fallback).
"""

from flare_amd.contracts import (
    SPARSE_EMBEDDING_OPERATOR_BACKENDS,
    SparseEmbeddingOperator,
    SparsePooledWidths,
    pooled_sparse_widths,
)
from flare_amd.factory import create_sparse_embedding_operator
from flare_amd.precision import prepare_sparse_native_gradient

__all__ = [
    "SPARSE_EMBEDDING_OPERATOR_BACKENDS",
    "SparseEmbeddingOperator",
    "SparsePooledWidths",
    "create_sparse_embedding_operator",
    "pooled_sparse_widths",
    "prepare_sparse_native_gradient",
]
