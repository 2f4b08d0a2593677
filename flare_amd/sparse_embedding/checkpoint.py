"""``sparse_embedding.checkpoint`` names the hot path imports.

``SUPPORTED_KEY_DTYPES`` feeds the key dtype contract
(``src/flare/runtime/sparse_precision.py:6,52-73``).  ``PartitionSpec`` and
``CheckpointSaveMode`` are the types the worker module imports at load time
(``src/flare/runtime/fluxway/workers/dynamic_embedding.py:7-10,805-806``); they
carry their values for those callers.  Key-owner routing across workers and
the checkpoint writer behind them are not part of this one-GPU store.
"""

from __future__ import annotations

import enum
from dataclasses import dataclass

SUPPORTED_KEY_DTYPES = frozenset({"int32", "uint32", "int64", "uint64"})


class CheckpointSaveMode(enum.Enum):
    FULL = "full"
    INCREMENTAL = "incremental"


@dataclass(frozen=True)
class PartitionSpec:
    """Key-owner assignment: ``key % owners`` (``modulo``) or a hash of the key (``hash``)."""

    kind: str

    @classmethod
    def modulo(cls) -> "PartitionSpec":
        return cls("modulo")

    @classmethod
    def hash(cls) -> "PartitionSpec":
        return cls("hash")


__all__ = ["CheckpointSaveMode", "PartitionSpec", "SUPPORTED_KEY_DTYPES"]
