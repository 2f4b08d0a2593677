"""The ``sparse_embedding`` store surface the sparse worker builds, over this library's HBM store.

``DynamicSparseEmbeddingSPMD`` constructs its store as
(``src/flare/runtime/fluxway/workers/dynamic_embedding.py:250-302``)::

    se.EmbeddingStore(
        embedding_config=se.EmbeddingConfig(dims=..., thread_budget=..., value_dtype=...,
                                            gradient_dtype=..., optimizer_dtype=..., key_dtype=...,
                                            storage=se.AutoStorage(...), enable_optimizer=...),
        initializer_config=se.Uniform(min_val=-0.01, max_val=0.01),
        optimizer_config=se.Adam(lr=..., ..., dynamic_lr_policy=se.ConstantLrPolicy()),
        score_policy="lfu",
    )

and drives it through ``reserve``, ``async_lookup_or_insert``,
``async_lookup``, ``async_accumulate_gradients`` and ``async_optimizer_step``
with DLPack capsules or arrays (``:296-302,396-400,512-527,538-546``).  This
module provides those names with the same arguments.  ``install()`` registers
it (and ``.checkpoint``) as the importable module ``sparse_embedding``, so the
worker's ``import sparse_embedding as se`` binds to it unchanged.

The store behind it is ``flare_amd.store.DynamicEmbeddingStore``: arbitrary
int64 keys, an HBM hash map per dim, rows and fp32 optimizer state in HBM, all
work on the store's HIP stream.  It grows by itself (``reserve`` grows it
ahead of time).  Deliberate limits, each raising ``ValueError`` where a caller
would depend on it: dynamic learning-rate policies other than constant,
``weight_decay != 0`` and ``score_policy`` values other than ``"lfu"``.  Rows
are never evicted (the LFU score only matters for eviction and spill, which
this store does not do); ``AutoStorage(memory_limit_bytes=...)`` caps the HBM
the tables may grow to.
"""

from __future__ import annotations

import sys
from dataclasses import dataclass, field
from typing import Any, Sequence

import numpy as np

from flare_amd.sparse_embedding import checkpoint


# ----------------------------------------------------------------------------
# learning-rate policies and optimizers (dynamic_embedding.py:69-106)
# ----------------------------------------------------------------------------
class LrPolicy:
    """Base of the dynamic learning-rate policies; only the constant one is implemented."""

    name = "policy"


class ConstantLrPolicy(LrPolicy):
    name = "constant"


class SqrtDecayLrPolicy(LrPolicy):
    name = "sqrt_decay"


class LogDecayLrPolicy(LrPolicy):
    name = "log_decay"


class InverseDecayLrPolicy(LrPolicy):
    name = "inverse_decay"


class CosineFrequencyLrPolicy(LrPolicy):
    name = "cosine_frequency"

    def __init__(self, min_lr_ratio: float = 0.0, max_score: Any = None):
        self.min_lr_ratio = min_lr_ratio
        self.max_score = max_score


class CustomLutLrPolicy(LrPolicy):
    name = "custom_lut"

    def __init__(self, lut: Any = None):
        self.lut = lut


class Optimizer:
    """Base of the optimizer configs (``se.Optimizer``)."""


def _policy_name(policy: Any) -> str:
    if policy is None:
        return "constant"
    if isinstance(policy, str):
        return policy
    return getattr(policy, "name", type(policy).__name__)


class Adam(Optimizer):
    """``se.Adam`` (``dynamic_embedding.py:89-96``); math of ``audit_sparse_training.py:460-471``."""

    def __init__(self, lr: float = 0.01, beta1: float = 0.9, beta2: float = 0.999, eps: float = 1e-8,
                 weight_decay: float = 0.0, dynamic_lr_policy: Any = None):
        self.lr, self.beta1, self.beta2, self.eps = float(lr), float(beta1), float(beta2), float(eps)
        self.weight_decay = float(weight_decay)
        self.dynamic_lr_policy = dynamic_lr_policy

    def _native(self):
        from flare_amd.store import Adam as _Adam

        return _Adam(self.lr, self.beta1, self.beta2, self.eps, self.weight_decay,
                     _policy_name(self.dynamic_lr_policy))


class Sgd(Optimizer):
    """``se.Sgd`` (``dynamic_embedding.py:97-101``): ``w -= lr * g``."""

    def __init__(self, lr: float = 0.01, weight_decay: float = 0.0, dynamic_lr_policy: Any = None):
        self.lr, self.weight_decay = float(lr), float(weight_decay)
        self.dynamic_lr_policy = dynamic_lr_policy

    def _native(self):
        from flare_amd.store import Sgd as _Sgd

        return _Sgd(self.lr, self.weight_decay, _policy_name(self.dynamic_lr_policy))


class RowWiseAdagrad(Optimizer):
    """One fp32 accumulator per row (no counterpart in the reference's store)."""

    def __init__(self, lr: float = 0.01, eps: float = 1e-8, initial_accumulator_value: float = 0.0):
        self.lr, self.eps = float(lr), float(eps)
        self.initial_accumulator_value = float(initial_accumulator_value)

    def _native(self):
        from flare_amd.store import RowWiseAdagrad as _R

        return _R(self.lr, self.eps, self.initial_accumulator_value)


# ----------------------------------------------------------------------------
# initializers, storage options, embedding config
# ----------------------------------------------------------------------------
@dataclass(frozen=True)
class Uniform:
    """``se.Uniform(min_val, max_val)`` (``dynamic_embedding.py:263``)."""

    min_val: float = -0.01
    max_val: float = 0.01


@dataclass(frozen=True)
class Zeros:
    pass


@dataclass(frozen=True)
class AutoStorage:
    """``se.AutoStorage`` (``src/flare/runtime/sparse_storage.py:40-46``): here the HBM cap."""

    memory_limit_bytes: int | None = None
    spill_directory: str | None = None
    max_spill_bytes: int | None = None


@dataclass(frozen=True)
class StorageTuningOptions:
    """``se.StorageTuningOptions`` (``sparse_storage.py:47-53``); pages do not apply to HBM tables."""

    max_pages: int = 0
    entries_per_page: int = 0
    calibrate_page_geometry: bool = True


@dataclass
class EmbeddingConfig:
    """``se.EmbeddingConfig`` as the worker fills it (``dynamic_embedding.py:251-260``)."""

    dims: Sequence[int] = field(default_factory=list)
    thread_budget: int = 1
    value_dtype: str = "float32"
    gradient_dtype: str = "float32"
    optimizer_dtype: str = "float32"
    key_dtype: str = "int64"
    storage: AutoStorage | None = None
    storage_tuning: StorageTuningOptions | None = None
    enable_optimizer: bool = True


_INITIAL_ROWS = 1 << 16


class EmbeddingStore:
    """``se.EmbeddingStore`` over ``DynamicEmbeddingStore`` (see the module docstring)."""

    def __init__(self, embedding_config: EmbeddingConfig, initializer_config: Any = None,
                 optimizer_config: Optimizer | None = None, score_policy: str = "lfu", *,
                 seed: int = 0, device: Any = None, initial_rows: int = _INITIAL_ROWS):
        from flare_amd.precision import require_key_dtype, require_sparse_optimizer_dtype
        from flare_amd.store import DynamicEmbeddingStore, Zeros as _Zeros, Uniform as _Uniform

        if not isinstance(embedding_config, EmbeddingConfig):
            raise TypeError(f"embedding_config must be EmbeddingConfig, got {type(embedding_config).__name__}")
        if score_policy != "lfu":
            raise ValueError(f"unsupported score_policy {score_policy!r} (only 'lfu')")
        dims = [int(d) for d in embedding_config.dims]
        if not dims or any(d <= 0 for d in dims):
            raise ValueError(f"embedding dims must be positive, got {embedding_config.dims!r}")
        require_key_dtype(embedding_config.key_dtype)
        require_sparse_optimizer_dtype(embedding_config.optimizer_dtype)
        if embedding_config.enable_optimizer and optimizer_config is None:
            raise ValueError("enable_optimizer=True requires an optimizer_config")
        self.config = embedding_config
        self._optimizer_enabled = bool(embedding_config.enable_optimizer)
        if isinstance(initializer_config, Zeros):
            init = _Zeros()
        elif initializer_config is None:
            init = _Uniform()
        else:
            init = _Uniform(float(initializer_config.min_val), float(initializer_config.max_val))
        native_opt = optimizer_config._native() if optimizer_config is not None else None
        storage = embedding_config.storage
        self._memory_limit = getattr(storage, "memory_limit_bytes", None) if storage is not None else None
        self._store = DynamicEmbeddingStore(int(initial_rows), dims, value_dtype=embedding_config.value_dtype,
                                            optimizer=native_opt if native_opt is not None else _sgd_placeholder(),
                                            initializer=init, seed=seed, device=device)
        # keys that may hold rows, per dim (an upper bound kept on the host; exact after a sync)
        self._bound = {d: 0 for d in dims}
        self._check_memory()

    # -- capacity -------------------------------------------------------------------
    def _row_bytes(self) -> int:
        s = self._store
        total = 0
        for table in s.tables.values():
            per_row = table.table.element_size() * table.dim
            for t in (table.state0, table.state1, table.step):
                if t is not None:
                    per_row += t.element_size() * (t.numel() // max(table.rows, 1))
            total += per_row + 32  # and two 16-byte map slots
        return total

    def _check_memory(self, rows: int | None = None) -> None:
        if self._memory_limit is None:
            return
        need = (rows if rows is not None else self._store.capacity) * self._row_bytes()
        if need > int(self._memory_limit):
            raise MemoryError(
                f"sparse store needs {need} bytes of HBM for {rows or self._store.capacity} rows per table, "
                f"above memory_limit_bytes={self._memory_limit} (this store does not spill)"
            )

    def _ensure_room(self, dim: int, n: int) -> None:
        """Grow ``dim``'s table before a lookup_or_insert of ``n`` keys could overflow it."""
        table = self._store._table(dim)
        bound = self._bound[dim] + n
        if bound > table.rows:
            count = self._store.size(dim)  # synchronizes: exact count
            bound = count + n
            if bound > table.rows:
                rows = max(2 * table.rows, bound)
                self._check_memory(rows)
                self._store.reserve(rows, dim)
        self._bound[dim] = bound

    def reserve(self, capacity: int, dim: int) -> None:
        capacity = int(capacity)
        if capacity < 0:
            raise ValueError(f"reserve capacity must be non-negative, got {capacity}")
        if capacity > self._store._table(dim).rows:
            self._check_memory(capacity)
        self._store.reserve(capacity, dim)

    # -- metadata -----------------------------------------------------------------------
    def value_dtype(self) -> str:
        return self._store.value_dtype()

    def optimizer_dtype(self) -> str:
        return "float32"

    def key_dtype(self) -> str:
        return self.config.key_dtype

    def optimizer_enabled(self) -> bool:
        return self._optimizer_enabled

    def table_dims(self) -> list[int]:
        return self._store.table_dims()

    def total_size(self) -> int:
        return self._store.size()

    def size(self, dim: int | None = None) -> int:
        return self._store.size(dim)

    def contains(self, keys: Any, dim: int | None = None) -> np.ndarray:
        return self._store.contains(keys, dim)

    def storage_stats(self) -> dict:
        """Rows held and HBM reserved per dim (synchronizes)."""
        stats = {}
        for dim, table in self._store.tables.items():
            stats[int(dim)] = {"keys": self._store.size(dim), "rows_reserved": table.rows,
                               "map_slots": self._store.maps[dim].slots}
        return stats

    # -- lookup ---------------------------------------------------------------------------
    def _keys(self, keys: Any):
        return self._store._keys(keys)

    def lookup_or_insert(self, keys: Any, dim: int):
        from flare_amd.array import DeviceArray

        k = self._keys(keys)
        self._ensure_room(int(dim), int(k.numel()))
        values, _ = self._store.lookup_or_insert(k, dim)
        return DeviceArray(values), None

    def lookup(self, keys: Any, dim: int):
        from flare_amd.array import DeviceArray

        values, _ = self._store.lookup(self._keys(keys), dim)
        return DeviceArray(values), None

    async def async_lookup_or_insert(self, keys: Any, dim: int):
        return self.lookup_or_insert(keys, dim)

    async def async_lookup(self, keys: Any, dim: int):
        return self.lookup(keys, dim)

    # -- update -------------------------------------------------------------------------------
    def _require_optimizer(self, what: str) -> None:
        if not self._optimizer_enabled:
            raise RuntimeError(f"{what} requires enable_optimizer=True")

    def accumulate_gradients(self, keys: Any, grad: Any) -> None:
        self._require_optimizer("accumulate_gradients")
        self._store.accumulate_gradients(keys, grad)

    def optimizer_step(self, normalization_steps: int) -> None:
        self._require_optimizer("optimizer_step")
        self._store.optimizer_step(normalization_steps)

    async def async_accumulate_gradients(self, keys: Any, grad: Any) -> None:
        self.accumulate_gradients(keys, grad)

    async def async_optimizer_step(self, normalization_steps: int) -> None:
        self.optimizer_step(normalization_steps)

    # -- checkpoint pages and assign --------------------------------------------------------------
    def export_page_images(self, page_keys: int = 1 << 20) -> list[dict]:
        return self._store.export_page_images(page_keys)

    def import_page_images(self, pages) -> None:
        pages = list(pages)
        for page in pages:
            dim = int(page["embedding_dim"])
            self._ensure_room(dim, int(np.asarray(page["keys"]).size))
        self._store.import_page_images(pages)

    def assign(self, keys: Any, values: Any) -> None:
        k = self._keys(keys)
        from flare_amd.conversion import to_device

        v = to_device(values, self._store.device)
        if v.dim() == 2:
            self._ensure_room(int(v.shape[1]), int(k.numel()))
        self._store.assign(k, v)

    def synchronize(self) -> None:
        self._store.synchronize()


def _sgd_placeholder():
    """Optimizer of a store built with enable_optimizer=False: no state; never stepped."""
    from flare_amd.store import Sgd as _Sgd

    return _Sgd(0.0)


def install() -> None:
    """Make ``import sparse_embedding`` (and ``sparse_embedding.checkpoint``) resolve here."""
    sys.modules["sparse_embedding"] = sys.modules[__name__]
    sys.modules["sparse_embedding.checkpoint"] = checkpoint


__all__ = [
    "Adam", "AutoStorage", "ConstantLrPolicy", "CosineFrequencyLrPolicy", "CustomLutLrPolicy", "EmbeddingConfig",
    "EmbeddingStore", "InverseDecayLrPolicy", "LogDecayLrPolicy", "LrPolicy", "Optimizer", "RowWiseAdagrad",
    "Sgd", "SqrtDecayLrPolicy", "StorageTuningOptions", "Uniform", "Zeros", "checkpoint", "install",
]
