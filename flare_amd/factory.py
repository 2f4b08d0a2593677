"""Operator factory (``src/flare/ops/factory.py:14-48``), same signature.

``"hip"`` selects the MI355X operator.  An unknown name raises ``ValueError``
listing the available backends, as the reference does (``factory.py:45-48``).
"""

from __future__ import annotations

from flare_amd.contracts import SPARSE_EMBEDDING_OPERATOR_BACKENDS, SparseEmbeddingOperator


def create_sparse_embedding_operator(
    name: str,
    *,
    value_dtype: str,
    gradient_dtype: str,
    empty_cache: bool = False,
    memory_reclaimer=None,
) -> SparseEmbeddingOperator:
    if name == "hip":
        from flare_amd.operator import HipSparseEmbeddingOperator

        return HipSparseEmbeddingOperator(
            value_dtype=value_dtype,
            gradient_dtype=gradient_dtype,
            empty_cache=empty_cache,
            memory_reclaimer=memory_reclaimer,
        )
    raise ValueError(
        f"Unknown sparse embedding operator backend {name!r}; "
        f"expected one of {SPARSE_EMBEDDING_OPERATOR_BACKENDS}."
    )
