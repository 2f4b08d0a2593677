"""HBM-resident sparse tables and their fused optimizer update.

``EmbeddingStore`` provides the subset of the external ``sparse_embedding``
store that ``DynamicSparseEmbeddingSPMD`` uses
(``src/flare/runtime/fluxway/workers/dynamic_embedding.py:251-302,397,525,544``):
``lookup_or_insert`` / ``lookup`` / ``accumulate_gradients`` /
``optimizer_step(normalization_steps)`` and their ``async_*`` forms,
``reserve``, ``value_dtype`` and ``optimizer_dtype``.  Keys are row indices of
a pre-sized dense shard ``[0, capacity)``; gradients accumulate per key until
``optimizer_step``, which divides the keyed sum by ``normalization_steps`` and
applies the optimizer (``dynamic_embedding.py:529-549``).

``PooledTableShard`` packs several tables of one worker into a single HBM
array and runs the fused hot path: CSR pooled lookup (forward) and
dedup + segment-reduce + optimizer update straight from pooled gradients
(backward), i.e. ``gather_pooled`` + ``scatter_pooled`` +
``accumulate_gradients`` + ``optimizer_step`` without materializing the
per-key gradients.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Any, Sequence

import numpy as np
import torch

from flare_amd import _native
from flare_amd.conversion import TORCH_VALUE_DTYPES, contiguous, storage_code, to_device
from flare_amd.precision import require_sparse_value_dtype

_POOLING = {"sum": _native.POOL_SUM, "mean": _native.POOL_MEAN, "weighted": _native.POOL_WEIGHTED}
_LAYOUTS = {"sample_major": _native.LAYOUT_SAMPLE_MAJOR, "table_major": _native.LAYOUT_TABLE_MAJOR}

# Gradient transport dtypes read as they are (SPARSE_GRADIENT_TRANSPORT_DTYPES,
# sparse_precision.py:12-14): bfloat16 widens to float32 on load, exactly.
_GRAD_TRANSPORT = {torch.float32: _native.FLOAT32, torch.bfloat16: _native.BFLOAT16}
_NONFINITE_MESSAGE = "non-finite sparse values at sparse_native_gradient"


def _transport_grad(g: torch.Tensor) -> torch.Tensor:
    """float32 and bfloat16 gradients are used as they are; others are cast to float32."""
    if g.dtype not in _GRAD_TRANSPORT:
        g = g.to(torch.float32)
    return contiguous(g)


def _raise_if_nonfinite(flag: torch.Tensor, stream: torch.cuda.Stream) -> None:
    """``require_finite_sparse_values`` (sparse_precision.py:121-148): reads the device flag."""
    stream.synchronize()
    if int(flag.item()):
        raise FloatingPointError(_NONFINITE_MESSAGE)


class _Ordered:
    """Runs a call's work on ``stream`` ordered against the caller's current stream.

    Entering makes ``stream`` wait for the caller's stream (inputs the caller
    is still producing there are complete before the store reads them) and
    makes ``stream`` current; leaving makes the caller's stream wait for
    ``stream`` (the results are ready for whatever the caller enqueues next).
    ``hold`` marks caller tensors the store reads or keeps as used by ``stream``
    and ``give`` marks results as used by the caller's stream, so the caching
    allocator reuses neither block while the other stream may still touch it.
    """

    def __init__(self, stream: torch.cuda.Stream, device: torch.device):
        self.stream = stream
        self.device = device
        self.caller: torch.cuda.Stream | None = None
        self._ctx = None

    def __enter__(self) -> "_Ordered":
        self.caller = torch.cuda.current_stream(self.device)
        if self.caller != self.stream:
            self.stream.wait_stream(self.caller)
        self._ctx = torch.cuda.stream(self.stream)
        self._ctx.__enter__()
        return self

    def __exit__(self, *exc) -> None:
        self._ctx.__exit__(*exc)
        if self.caller != self.stream:
            self.caller.wait_stream(self.stream)

    def hold(self, *tensors: Any) -> None:
        for t in tensors:
            if isinstance(t, torch.Tensor) and t.device.type == "cuda":
                t.record_stream(self.stream)

    def give(self, *tensors: Any) -> None:
        for t in tensors:
            if isinstance(t, torch.Tensor) and t.device.type == "cuda" and self.caller != self.stream:
                t.record_stream(self.caller)


# ----------------------------------------------------------------------------
# optimizer and initializer configs (se.Adam / se.Sgd / se.Uniform / se.Zeros)
# ----------------------------------------------------------------------------
@dataclass(frozen=True)
class Adam:
    """``se.Adam`` (dynamic_embedding.py:89-96); math of audit_sparse_training.py:460-471."""

    lr: float = 0.01
    beta1: float = 0.9
    beta2: float = 0.999
    eps: float = 1e-8
    weight_decay: float = 0.0
    dynamic_lr_policy: str = "constant"


@dataclass(frozen=True)
class Sgd:
    """``se.Sgd`` (dynamic_embedding.py:97-101): ``w -= lr * g``."""

    lr: float = 0.01
    weight_decay: float = 0.0
    dynamic_lr_policy: str = "constant"


@dataclass(frozen=True)
class RowWiseAdagrad:
    """One fp32 accumulator per row: ``acc += mean(g^2); w -= lr*g/(sqrt(acc)+eps)``."""

    lr: float = 0.01
    eps: float = 1e-8
    initial_accumulator_value: float = 0.0


@dataclass(frozen=True)
class Uniform:
    """``se.Uniform`` (the worker's default is ``Uniform(-0.01, 0.01)``, dynamic_embedding.py:263)."""

    min_val: float = -0.01
    max_val: float = 0.01


@dataclass(frozen=True)
class Zeros:
    pass


def optimizer_from_config(config: Any):
    """Map a ``SparseOptimizerConfig``-like object (sparse_table/contracts.py:14-25)."""
    kind = getattr(config, "kind", "adam")
    policy = getattr(config, "dynamic_lr_policy", "constant")
    if kind == "adam":
        return Adam(config.learning_rate, config.beta1, config.beta2, config.eps,
                    config.weight_decay, policy)
    if kind == "sgd":
        return Sgd(config.learning_rate, config.weight_decay, policy)
    if kind in ("rowwise_adagrad", "adagrad"):
        return RowWiseAdagrad(config.learning_rate, config.eps)
    raise ValueError(f"unsupported sparse optimizer {kind!r}")


def _native_optimizer(optimizer: Any) -> _native.FlareOptimizer:
    if getattr(optimizer, "dynamic_lr_policy", "constant") != "constant":
        raise ValueError(
            "unsupported sparse dynamic learning-rate policy "
            f"{optimizer.dynamic_lr_policy!r} (only 'constant' is implemented)"
        )
    if getattr(optimizer, "weight_decay", 0.0) != 0.0:
        raise ValueError("sparse optimizer weight_decay must be 0")
    o = _native.FlareOptimizer()
    o.learning_rate = float(optimizer.lr)
    o.eps = float(getattr(optimizer, "eps", 0.0))
    o.beta1 = float(getattr(optimizer, "beta1", 0.0))
    o.beta2 = float(getattr(optimizer, "beta2", 0.0))
    o.weight_decay = 0.0
    if isinstance(optimizer, Adam):
        o.kind = _native.OPT_ADAM
    elif isinstance(optimizer, Sgd):
        o.kind = _native.OPT_SGD
    elif isinstance(optimizer, RowWiseAdagrad):
        o.kind = _native.OPT_ROWWISE_ADAGRAD
    elif optimizer is None:
        o.kind = _native.OPT_NONE
    else:
        raise TypeError(f"unsupported sparse optimizer config {type(optimizer).__name__}")
    return o


# ----------------------------------------------------------------------------
# one dense table with its optimizer state
# ----------------------------------------------------------------------------
class _TableState:
    def __init__(self, rows: int, dim: int, value_dtype: str, optimizer: Any,
                 initializer: Any, generator: torch.Generator, device: torch.device):
        self.rows, self.dim = int(rows), int(dim)
        self.value_dtype = require_sparse_value_dtype(value_dtype)
        dtype = TORCH_VALUE_DTYPES[value_dtype]
        if isinstance(initializer, Zeros):
            table = torch.zeros((self.rows, self.dim), dtype=torch.float32, device=device)
        else:
            init = initializer or Uniform()
            table = torch.empty((self.rows, self.dim), dtype=torch.float32, device=device)
            table.uniform_(float(init.min_val), float(init.max_val), generator=generator)
        # fp32 -> storage rounds to nearest even
        self.table = table.to(dtype)
        del table
        self.optimizer = optimizer
        self.state0 = self.state1 = self.step = None
        if isinstance(optimizer, Adam):
            self.state0 = torch.zeros((self.rows, self.dim), dtype=torch.float32, device=device)
            self.state1 = torch.zeros((self.rows, self.dim), dtype=torch.float32, device=device)
            self.step = torch.zeros(self.rows, dtype=torch.int32, device=device)
        elif isinstance(optimizer, RowWiseAdagrad):
            self.state0 = torch.full((self.rows,), float(optimizer.initial_accumulator_value),
                                     dtype=torch.float32, device=device)
        self.native_optimizer = _native_optimizer(optimizer)

    def pointers(self):
        p = lambda t: None if t is None else t.data_ptr()  # noqa: E731
        return p(self.state0), p(self.state1), p(self.step)

    def grow(self, rows: int) -> None:
        """Room for ``rows`` rows: existing rows and state are kept, new rows are zero (state
        at its initial value)."""
        rows = int(rows)
        if rows <= self.rows:
            return

        def bigger(t: torch.Tensor | None, fill: float = 0.0) -> torch.Tensor | None:
            if t is None:
                return None
            out = torch.full((rows,) + tuple(t.shape[1:]), fill, dtype=t.dtype, device=t.device)
            out[: t.shape[0]].copy_(t)
            return out

        self.table = bigger(self.table)
        fill0 = float(getattr(self.optimizer, "initial_accumulator_value", 0.0))
        self.state0 = bigger(self.state0, fill0 if isinstance(self.optimizer, RowWiseAdagrad) else 0.0)
        self.state1 = bigger(self.state1)
        self.step = bigger(self.step)
        self.rows = rows


class _Workspace:
    """Grow-only device scratch owned by one stream."""

    def __init__(self, device: torch.device):
        self.device = device
        self.buffer: torch.Tensor | None = None

    def get(self, nbytes: int) -> torch.Tensor:
        nbytes = max(int(nbytes), 1)
        if self.buffer is None or self.buffer.numel() < nbytes:
            self.buffer = None
            self.buffer = torch.empty(nbytes, dtype=torch.uint8, device=self.device)
        return self.buffer


def _device_of(device: Any) -> torch.device:
    if device is None:
        return torch.device("cuda", torch.cuda.current_device())
    return torch.device(device)


# ----------------------------------------------------------------------------
# EmbeddingStore
# ----------------------------------------------------------------------------
class EmbeddingStore:
    """Dense row-indexed store, one table per embedding dim, resident in HBM."""

    def __init__(self, capacity: int, dims: Sequence[int], *, value_dtype: str = "float32",
                 optimizer: Any = None, initializer: Any = None, seed: int = 0,
                 device: Any = None, validate_values: bool = False):
        if not torch.cuda.is_available():
            raise RuntimeError("EmbeddingStore requires a ROCm GPU")
        if not isinstance(validate_values, bool):
            raise TypeError("validate_values must be bool")
        self.validate_values = validate_values
        _native.library()
        self.device = _device_of(device)
        self.capacity = int(capacity)
        self._value_dtype = require_sparse_value_dtype(value_dtype)
        self.stream = torch.cuda.Stream(device=self.device)
        generator = torch.Generator(device=self.device)
        generator.manual_seed(int(seed))
        with torch.cuda.stream(self.stream):
            self.tables = {
                int(d): _TableState(self.capacity, int(d), value_dtype, optimizer or Adam(),
                                    initializer, generator, self.device)
                for d in dims
            }
        self._pending: dict[int, list[tuple[torch.Tensor, torch.Tensor]]] = {}
        self._workspace = _Workspace(self.device)
        torch.cuda.current_stream(self.device).wait_stream(self.stream)  # tables initialized

    # -- metadata -------------------------------------------------------------
    def value_dtype(self) -> str:
        return self._value_dtype

    def optimizer_dtype(self) -> str:
        return "float32"

    def total_size(self) -> int:
        return self.capacity * len(self.tables)

    def reserve(self, capacity: int, dim: int) -> None:
        self._table(dim)
        if int(capacity) > self.capacity:
            raise ValueError(
                f"dense sparse shard holds {self.capacity} rows; cannot reserve {capacity}"
            )

    def contains(self, keys: Any) -> np.ndarray:
        k = np.asarray(keys, dtype=np.int64)
        return (k >= 0) & (k < self.capacity)

    def _table(self, dim: int) -> _TableState:
        try:
            return self.tables[int(dim)]
        except KeyError as error:
            raise ValueError(f"store has no table of dim {dim}") from error

    def _keys(self, keys: Any) -> torch.Tensor:
        k = to_device(keys, self.device)
        if k.dtype not in (torch.int64, torch.int32):
            raise TypeError(f"sparse keys must be int64 (or int32), got {k.dtype}")
        return contiguous(k.reshape(-1).to(torch.int64))

    # -- lookup ---------------------------------------------------------------
    def lookup(self, keys: Any, dim: int):
        """Rows of ``keys`` as a ``[n, dim]`` tensor of the value dtype (DLPack producer)."""
        table = self._table(dim)
        with _Ordered(self.stream, self.device) as order:
            k = self._keys(keys)
            order.hold(k)
            out = torch.empty((k.numel(), table.dim), dtype=table.table.dtype, device=self.device)
            if k.numel():
                inv = contiguous(torch.clamp(k, -1, table.rows).to(torch.int32))
                _native.call(
                    "flare_gather", table.table.data_ptr(), storage_code(table.table.dtype),
                    table.rows, table.dim, inv.data_ptr(), k.numel(), table.rows + 1,
                    out.data_ptr(), int(self.stream.cuda_stream),
                )
            order.give(out)
        return out, None

    def lookup_or_insert(self, keys: Any, dim: int):
        """Dense shard: every key in ``[0, capacity)`` already has a row."""
        return self.lookup(keys, dim)

    # -- update ---------------------------------------------------------------
    def accumulate_gradients(self, keys: Any, grad: Any) -> None:
        """Keyed gradients in float32 or bfloat16 transport (others are cast to float32).  With
        ``validate_values`` a non-finite gradient raises ``FloatingPointError`` here, before
        anything accumulates (synchronizes)."""
        with _Ordered(self.stream, self.device) as order:
            k = self._keys(keys)
            g = _transport_grad(to_device(grad, self.device))
            order.hold(k, g)  # kept in _pending until optimizer_step
            if g.dim() != 2 or g.shape[0] != k.numel():
                raise ValueError(
                    f"gradient shape {tuple(g.shape)} does not match {k.numel()} keys"
                )
            self._table(g.shape[1])
            if self.validate_values and g.numel():
                flag = torch.empty(1, dtype=torch.int32, device=self.device)
                _native.call("flare_check_finite", g.data_ptr(), _GRAD_TRANSPORT[g.dtype], g.numel(),
                             flag.data_ptr(), int(self.stream.cuda_stream))
                _raise_if_nonfinite(flag, self.stream)
            self._pending.setdefault(int(g.shape[1]), []).append((k, g))

    def optimizer_step(self, normalization_steps: int) -> None:
        if isinstance(normalization_steps, bool) or not isinstance(normalization_steps, int) or normalization_steps <= 0:
            raise ValueError("normalization_steps must be a positive integer")
        with _Ordered(self.stream, self.device):
            for dim, items in self._pending.items():
                table = self._table(dim)
                keys = items[0][0] if len(items) == 1 else torch.cat([k for k, _ in items])
                if all(g.dtype == torch.bfloat16 for _, g in items):
                    grad = items[0][1] if len(items) == 1 else torch.cat([g for _, g in items])
                else:  # one dtype per call: mixed windows are widened to float32
                    grad = items[0][1] if len(items) == 1 else torch.cat([g.to(torch.float32) for _, g in items])
                n = int(keys.numel())
                if n == 0:
                    continue
                nbytes = _native.library().flare_sparse_update_workspace_bytes(n, table.rows, table.dim)
                ws = self._workspace.get(nbytes)
                s0, s1, st = table.pointers()
                _native.call(
                    "flare_sparse_update_ex", table.table.data_ptr(), storage_code(table.table.dtype),
                    table.rows, table.dim, s0, s1, st, ctypes.byref(table.native_optimizer),
                    keys.data_ptr(), n, grad.data_ptr(), _GRAD_TRANSPORT[grad.dtype], 0, None,
                    int(normalization_steps), ws.data_ptr(), nbytes, int(self.stream.cuda_stream),
                )
            self._pending.clear()

    # -- checkpoint page images and assign ---------------------------------------
    # Page images as the reference's store hands them to its checkpoint code
    # (tests/runtime/test_sparse_storage_limits.py:62-79,
    # tools/validation/audit_sparse_checkpoint.py:33-70): per page the
    # embedding dim, keys (uint64 view of int64), values [n * dim], optimizer
    # states [n * width] (Adam: m then v, 2 * dim; row-wise Adagrad: the
    # accumulator, 1; SGD: none) and per-key update steps (uint32; counted for
    # Adam only, 0 otherwise).  bfloat16 values are exported as float32.
    def optimizer_enabled(self) -> bool:
        return True

    def table_dims(self) -> list[int]:
        return list(self.tables)

    def key_dtype(self) -> str:
        return "int64"

    def num_slots(self) -> int:
        return len(self.tables)

    def _rows_of(self, keys: torch.Tensor, dim: int, insert: bool) -> torch.Tensor:
        """Rows of keys (int32): the keys themselves in the dense shard."""
        table = self._table(dim)
        return contiguous(torch.clamp(keys, -1, table.rows).to(torch.int32))

    def _copy_rows(self, src: torch.Tensor, dst: torch.Tensor, src_index, dst_index, n: int) -> None:
        row_bytes = src.element_size() * (src[0].numel() if src.dim() > 1 else 1)
        p = lambda t: None if t is None else t.data_ptr()  # noqa: E731
        _native.call("flare_copy_rows", src.data_ptr(), src.shape[0], dst.data_ptr(), dst.shape[0], row_bytes,
                     p(src_index), p(dst_index), n, int(self.stream.cuda_stream))

    def _page(self, table: _TableState, keys: torch.Tensor, rows: torch.Tensor) -> dict:
        n = int(rows.numel())
        dev = self.device
        values = torch.empty((n, table.dim), dtype=table.table.dtype, device=dev)
        self._copy_rows(table.table, values, rows, None, n)
        opt = table.optimizer
        if isinstance(opt, Adam):
            state = torch.empty((n, 2 * table.dim), dtype=torch.float32, device=dev)
            m = torch.empty((n, table.dim), dtype=torch.float32, device=dev)
            v = torch.empty((n, table.dim), dtype=torch.float32, device=dev)
            self._copy_rows(table.state0, m, rows, None, n)
            self._copy_rows(table.state1, v, rows, None, n)
            state[:, : table.dim] = m
            state[:, table.dim:] = v
            steps = torch.empty(n, dtype=torch.int32, device=dev)
            self._copy_rows(table.step, steps, rows, None, n)
        elif isinstance(opt, RowWiseAdagrad):
            state = torch.empty((n, 1), dtype=torch.float32, device=dev)
            self._copy_rows(table.state0, state, rows, None, n)
            steps = torch.zeros(n, dtype=torch.int32, device=dev)
        else:
            state = torch.empty((n, 0), dtype=torch.float32, device=dev)
            steps = torch.zeros(n, dtype=torch.int32, device=dev)
        if values.dtype == torch.bfloat16:
            values = values.to(torch.float32)
        # device -> host into pinned buffers (about 50 GB/s, against about 4 GB/s for
        # pageable ones); the page's numpy arrays keep their buffers alive
        host = [_pinned_copy(t) for t in (keys, values, state, steps)]
        self.stream.synchronize()
        return {
            "embedding_dim": table.dim,
            "keys": host[0].numpy().view(np.uint64),
            "values": host[1].numpy().reshape(-1),
            "optimizer_states": host[2].numpy().reshape(-1),
            "steps": host[3].numpy().view(np.uint32),
        }

    def _stored(self, dim: int):
        """(keys int64, rows int32) of every stored key of ``dim``'s table, on the device."""
        table = self._table(dim)
        rows = torch.arange(table.rows, dtype=torch.int32, device=self.device)
        return rows.to(torch.int64), rows

    def export_page_images(self, page_keys: int = 1 << 20) -> list[dict]:
        pages = []
        with _Ordered(self.stream, self.device):
            for dim, table in self.tables.items():
                keys, rows = self._stored(dim)
                for lo in range(0, int(keys.numel()), int(page_keys)):
                    hi = min(lo + int(page_keys), int(keys.numel()))
                    pages.append(self._page(table, keys[lo:hi], contiguous(rows[lo:hi])))
        return pages

    def import_page_images(self, pages) -> None:
        """Writes every page's rows (values, optimizer state, steps) for its keys."""
        with _Ordered(self.stream, self.device):
            for page in pages:
                dim = int(page["embedding_dim"])
                table = self._table(dim)
                keys = torch.from_numpy(np.asarray(page["keys"], dtype=np.uint64).view(np.int64).copy()).to(self.device)
                n = int(keys.numel())
                if n == 0:
                    continue
                rows = self._rows_of(keys, dim, insert=True)
                values = torch.from_numpy(np.asarray(page["values"]).reshape(n, dim)).to(self.device)
                self._copy_rows(contiguous(values.to(table.table.dtype)), table.table, None, rows, n)
                state = np.asarray(page["optimizer_states"], dtype=np.float32).reshape(n, -1)
                if isinstance(table.optimizer, Adam):
                    st = torch.from_numpy(state).to(self.device)
                    self._copy_rows(contiguous(st[:, :dim]), table.state0, None, rows, n)
                    self._copy_rows(contiguous(st[:, dim:]), table.state1, None, rows, n)
                    steps = torch.from_numpy(np.asarray(page["steps"], dtype=np.uint32).view(np.int32).copy())
                    self._copy_rows(steps.to(self.device), table.step, None, rows, n)
                elif isinstance(table.optimizer, RowWiseAdagrad):
                    self._copy_rows(torch.from_numpy(state[:, :1].copy()).to(self.device), table.state0, None, rows, n)
        self.stream.synchronize()

    def assign(self, keys: Any, values: Any) -> None:
        """Sets the rows of ``keys`` (inserting them in a dynamic store) to ``values [n, dim]``."""
        with _Ordered(self.stream, self.device) as order:
            v = to_device(values, self.device)
            order.hold(v)
            if v.dim() != 2:
                raise ValueError(f"assign needs values of shape [keys, dim], got {tuple(v.shape)}")
            table = self._table(int(v.shape[1]))
            k = self._keys(keys)
            order.hold(k)
            if v.shape[0] != k.numel():
                raise ValueError(f"values shape {tuple(v.shape)} does not match {k.numel()} keys")
            rows = self._rows_of(k, table.dim, insert=True)
            self._copy_rows(contiguous(v.to(table.table.dtype)), table.table, None, rows, int(k.numel()))

    # -- async forms (work is enqueued on the store's stream either way) ------
    async def async_lookup_or_insert(self, keys: Any, dim: int):
        return self.lookup_or_insert(keys, dim)

    async def async_lookup(self, keys: Any, dim: int):
        return self.lookup(keys, dim)

    async def async_accumulate_gradients(self, keys: Any, grad: Any) -> None:
        self.accumulate_gradients(keys, grad)

    async def async_optimizer_step(self, normalization_steps: int) -> None:
        self.optimizer_step(normalization_steps)

    def synchronize(self) -> None:
        self.stream.synchronize()


# ----------------------------------------------------------------------------
# DynamicEmbeddingStore: arbitrary int64 keys through an HBM key -> row map
# ----------------------------------------------------------------------------
def _pinned_copy(t: torch.Tensor) -> torch.Tensor:
    """A pinned host copy of device tensor ``t``, enqueued on the current stream."""
    h = torch.empty(t.shape, dtype=t.dtype, pin_memory=True)
    h.copy_(t, non_blocking=True)
    return h


def _map_slots(rows: int) -> int:
    """Power-of-two slot count keeping the map at most half full."""
    slots = 64
    while slots < 2 * int(rows):
        slots *= 2
    return slots


class _KeyMap:
    def __init__(self, slots: int, device: torch.device, stream: torch.cuda.Stream):
        self.slots = int(slots)
        nbytes = _native.library().flare_keymap_bytes(self.slots)
        if nbytes == 0:
            raise ValueError(f"key map of {slots} slots is not supported (at most 2^30)")
        self.buffer = torch.empty(nbytes, dtype=torch.uint8, device=device)
        _native.call("flare_keymap_init", self.buffer.data_ptr(), self.slots, int(stream.cuda_stream))

    def count(self) -> int:
        """Keys holding a row (reads the header: synchronizes)."""
        return int(self.buffer[:4].view(torch.int32).item())


class DynamicEmbeddingStore(EmbeddingStore):
    """``EmbeddingStore`` over arbitrary int64 keys (INT64_MIN excepted).

    One HBM hash map per dim sends keys to rows of that dim's table.
    ``lookup_or_insert`` gives new keys rows in the order of their first
    occurrence and initial values ``Uniform(min_val, max_val)`` drawn from a
    counter-based hash of ``(seed, key, column)``, so a key's initial row does
    not depend on the batch it first arrives in (the worker's store,
    ``dynamic_embedding.py:251-302``, draws new rows from
    ``se.Uniform(-0.01, 0.01)``, ``:262-263``).  Rows are never evicted:
    ``reserve`` grows the table and the map; a full table sets device error
    bit 4 and returns zero rows for the keys left out.
    """

    def __init__(self, capacity: int, dims: Sequence[int], *, value_dtype: str = "float32",
                 optimizer: Any = None, initializer: Any = None, seed: int = 0,
                 device: Any = None):
        init = initializer or Uniform()
        if isinstance(init, Zeros):
            self._init_range = (0.0, 0.0)
        else:
            self._init_range = (float(init.min_val), float(init.max_val))
        self._seed = int(seed) & 0xFFFFFFFFFFFFFFFF
        super().__init__(capacity, dims, value_dtype=value_dtype, optimizer=optimizer,
                         initializer=Zeros(), seed=seed, device=device)
        with torch.cuda.stream(self.stream):
            self.maps = {d: _KeyMap(_map_slots(self.capacity), self.device, self.stream) for d in self.tables}
        self._map_workspace = _Workspace(self.device)
        self._row_bases: dict[int, tuple[int, torch.Tensor]] = {}  # dim -> (rows, [0, rows] on the device)
        torch.cuda.current_stream(self.device).wait_stream(self.stream)

    # -- keys -> rows -----------------------------------------------------------
    def _resolve(self, keys: torch.Tensor, dim: int, insert: bool, values: bool):
        table = self._table(dim)
        kmap = self.maps[int(dim)]
        n = int(keys.numel())
        rows = torch.empty(max(n, 1), dtype=torch.int32, device=self.device)
        out = torch.empty((n, table.dim), dtype=table.table.dtype, device=self.device) if values else None
        if n:
            nbytes = _native.library().flare_keymap_workspace_bytes(n)
            ws = self._map_workspace.get(nbytes)
            lo, hi = self._init_range
            _native.call(
                "flare_keymap_lookup_or_insert", kmap.buffer.data_ptr(), kmap.slots, keys.data_ptr(), n,
                1 if insert else 0, table.table.data_ptr(), storage_code(table.table.dtype), table.rows,
                table.dim, lo, hi, self._seed, rows.data_ptr(), None if out is None else out.data_ptr(),
                ws.data_ptr(), nbytes, int(self.stream.cuda_stream),
            )
        return rows[:n], out

    def rows(self, keys: Any, dim: int, *, insert: bool = False) -> torch.Tensor:
        """Row of every key in ``dim``'s table (int32, -1 when absent)."""
        with _Ordered(self.stream, self.device) as order:
            k = self._keys(keys)
            order.hold(k)
            rows = self._resolve(k, dim, insert, values=False)[0]
            order.give(rows)
            return rows

    def _values(self, keys: Any, dim: int, insert: bool):
        with _Ordered(self.stream, self.device) as order:
            k = self._keys(keys)
            order.hold(k)
            out = self._resolve(k, dim, insert, values=True)[1]
            order.give(out)
            return out, None

    def lookup(self, keys: Any, dim: int):
        """Rows of present keys, zeros for absent ones (``[n, dim]``, value dtype)."""
        return self._values(keys, dim, False)

    def lookup_or_insert(self, keys: Any, dim: int):
        return self._values(keys, dim, True)

    def contains(self, keys: Any, dim: int | None = None) -> np.ndarray:
        d = next(iter(self.tables)) if dim is None else int(dim)
        rows = self.rows(keys, d)
        self.stream.synchronize()
        return rows.cpu().numpy() >= 0

    def size(self, dim: int | None = None) -> int:
        """Keys holding a row in ``dim``'s table (all tables when None); synchronizes."""
        self.stream.synchronize()
        if dim is not None:
            return self.maps[int(dim)].count()
        return sum(m.count() for m in self.maps.values())

    def total_size(self) -> int:
        return self.size()

    def reserve(self, capacity: int, dim: int) -> None:
        table = self._table(dim)
        capacity = int(capacity)
        if capacity <= table.rows:
            return
        with _Ordered(self.stream, self.device):
            table.grow(capacity)
            old = self.maps[int(dim)]
            slots = _map_slots(capacity)
            if slots > old.slots:
                new = _KeyMap(slots, self.device, self.stream)
                _native.call("flare_keymap_rehash", old.buffer.data_ptr(), old.slots, new.buffer.data_ptr(),
                             new.slots, int(self.stream.cuda_stream))
                self.maps[int(dim)] = new
        self.capacity = max(self.capacity, capacity)

    def _rows_of(self, keys: torch.Tensor, dim: int, insert: bool) -> torch.Tensor:
        return self._resolve(keys, dim, insert, values=False)[0]

    def _stored(self, dim: int):
        kmap = self.maps[int(dim)]
        count = kmap.count()  # synchronizes
        keys = torch.empty(max(count, 1), dtype=torch.int64, device=self.device)
        rows = torch.empty(max(count, 1), dtype=torch.int32, device=self.device)
        total = torch.empty(1, dtype=torch.int64, device=self.device)
        nbytes = _native.library().flare_keymap_export_workspace_bytes(kmap.slots)
        ws = self._map_workspace.get(nbytes)
        _native.call("flare_keymap_export", kmap.buffer.data_ptr(), kmap.slots, keys.data_ptr(), rows.data_ptr(),
                     total.data_ptr(), ws.data_ptr(), nbytes, int(self.stream.cuda_stream))
        self.stream.synchronize()
        if int(total.item()) != count:
            raise RuntimeError(f"key map export found {int(total.item())} keys, expected {count}")
        return keys[:count], rows[:count]

    # -- gradients are kept per row ----------------------------------------------
    def accumulate_gradients(self, keys: Any, grad: Any) -> None:
        """Keys must have rows (looked up or inserted before); others set device error bit 1
        and their gradient is dropped at ``optimizer_step``."""
        with _Ordered(self.stream, self.device) as order:
            g = to_device(grad, self.device)
            if g.dim() != 2:
                raise ValueError(f"gradient must be [keys, dim], got shape {tuple(g.shape)}")
            k = self._keys(keys)
            order.hold(g, k)
            if g.shape[0] != k.numel():
                raise ValueError(f"gradient shape {tuple(g.shape)} does not match {k.numel()} keys")
            rows = self._resolve(k, int(g.shape[1]), False, values=False)[0].to(torch.int64)
        super().accumulate_gradients(rows, g)

    # -- the fused pooled step over keys ----------------------------------------
    # The reference materializes one feature group as keys -> unique keys ->
    # lookup_or_insert of the unique keys (dynamic_embedding.py:397-399) ->
    # gather_pooled of the compact rows by the padded inverse
    # (materialization.py:36-79), and on the way back scatter_pooled -> keyed sums
    # -> accumulate_gradients + optimizer_step (dynamic_embedding.py:481-549).
    # Here every occurrence's key goes through the key map once (rows in
    # first-occurrence order, new rows initialised), and the rows feed the fused
    # CSR kernels over this dim's table directly: T features of B bags, bag
    # k = t*B + b, pooled rows [T, B, D] (the [B, 1, D] outputs of T
    # single-feature groups, one after the other).
    def _pooled_keys(self, keys: Any, offsets: Any, batch_size: int, dim: int):
        table = self._table(dim)
        batch_size = int(batch_size)
        k = self._keys(keys)
        off = contiguous(to_device(offsets, self.device).reshape(-1).to(torch.int64))
        if batch_size <= 0 or (off.numel() - 1) % batch_size != 0 or off.numel() < 2:
            raise ValueError(f"offsets must hold features * batch_size + 1 entries, got {off.numel()} "
                             f"for batch_size {batch_size}")
        return table, k, off, (off.numel() - 1) // batch_size

    def _pooled_weights(self, pooling: str, per_sample_weights: Any, n: int):
        if pooling not in _POOLING:
            raise ValueError(f"pooling must be one of {sorted(_POOLING)}, got {pooling!r}")
        if pooling != "weighted":
            return None
        if per_sample_weights is None:
            raise ValueError("weighted pooling requires per_sample_weights")
        w = contiguous(to_device(per_sample_weights, self.device).reshape(-1).to(torch.float32))
        if w.numel() != n:
            raise ValueError("per_sample_weights must have one weight per key")
        return w

    def _one_table(self, table: _TableState) -> torch.Tensor:
        """row_base of the whole table as one CSR table: [0, rows] (kept until the table grows)."""
        hit = self._row_bases.get(table.dim)
        if hit is None or hit[0] != table.rows:
            base = torch.tensor([0, table.rows], dtype=torch.int64).pin_memory()
            hit = (table.rows, base.to(self.device, non_blocking=True))
            self._row_bases[table.dim] = hit
        return hit[1]

    def lookup_pooled(self, keys: Any, offsets: Any, batch_size: int, dim: int, *, pooling: str = "sum",
                      per_sample_weights: Any = None) -> torch.Tensor:
        """Forward over keys: ``lookup_or_insert`` of every key of the CSR bags, then the pooled
        gather of their rows; ``[features, batch_size, dim]`` in the value dtype."""
        with _Ordered(self.stream, self.device) as order:
            table, k, off, features = self._pooled_keys(keys, offsets, batch_size, dim)
            n = int(k.numel())
            w = self._pooled_weights(pooling, per_sample_weights, n)
            order.hold(k, off, w)
            rows = self._resolve(k, dim, True, values=False)[0] if n else \
                torch.empty(1, dtype=torch.int32, device=self.device)
            out = torch.empty((features, int(batch_size), table.dim), dtype=table.table.dtype, device=self.device)
            row_base = self._one_table(table)
            _native.call(
                "flare_gather_pooled_csr", table.table.data_ptr(), storage_code(table.table.dtype), table.rows,
                table.dim, rows.data_ptr(), _native.INT32, n, off.data_ptr(), 1, features * int(batch_size),
                row_base.data_ptr(), _POOLING[pooling], _native.LAYOUT_TABLE_MAJOR,
                None if w is None else w.data_ptr(), out.data_ptr(), int(self.stream.cuda_stream),
            )
            order.give(out)
        return out

    def apply_pooled_gradients(self, keys: Any, offsets: Any, batch_size: int, pooled_grad: Any, dim: int, *,
                               pooling: str = "sum", per_sample_weights: Any = None,
                               normalization_steps: int = 1, return_dedup: bool = False,
                               validate_values: bool = False):
        """Backward + update over keys: the rows of the keys (looked up, not inserted: keys without
        a row set device error bit 1 and are left out), then the fused dedup, deterministic
        segment sum and optimizer update of this dim's table.  ``pooled_grad``: float32 or
        bfloat16 ``[features, batch_size, dim]``.  With ``return_dedup`` also returns
        ``(unique_keys, inverse, first_indices)`` in first-occurrence order (synchronizes)."""
        if isinstance(normalization_steps, bool) or not isinstance(normalization_steps, int) or \
                normalization_steps <= 0:
            raise ValueError("normalization_steps must be a positive integer")
        with _Ordered(self.stream, self.device) as order:
            table, k, off, features = self._pooled_keys(keys, offsets, batch_size, dim)
            n = int(k.numel())
            w = self._pooled_weights(pooling, per_sample_weights, n)
            g = _transport_grad(to_device(pooled_grad, self.device))
            order.hold(k, off, w, g)
            bags = features * int(batch_size)
            if g.numel() != bags * table.dim or not g.is_contiguous():
                raise ValueError(f"pooled gradient must be a contiguous [{features}, {batch_size}, {table.dim}] "
                                 "tensor")
            rows = self._resolve(k, dim, False, values=False)[0] if n else \
                torch.empty(1, dtype=torch.int32, device=self.device)
            row_base = self._one_table(table)
            m = max(n, 1)
            unique = torch.empty(m, dtype=torch.int64, device=self.device)
            first = torch.empty(m, dtype=torch.int64, device=self.device)
            inverse = torch.empty(m, dtype=torch.int32, device=self.device)
            count = torch.zeros(1, dtype=torch.int64, device=self.device)
            flag = torch.zeros(1, dtype=torch.int32, device=self.device) if validate_values else None
            nbytes = _native.library().flare_pooled_backward_workspace_bytes(n, table.rows, table.dim)
            ws = self._workspace.get(nbytes)
            s0, s1, st = table.pointers()
            stream = int(self.stream.cuda_stream)
            _native.call(
                "flare_pooled_dedup", rows.data_ptr(), _native.INT32, n, off.data_ptr(), 1, bags,
                row_base.data_ptr(), table.rows, table.dim, _POOLING[pooling], _native.LAYOUT_TABLE_MAJOR,
                unique.data_ptr(), first.data_ptr(), count.data_ptr(), ws.data_ptr(), nbytes, stream,
            )
            _native.call(
                "flare_pooled_apply_ex", table.table.data_ptr(), storage_code(table.table.dtype), table.rows,
                table.dim, s0, s1, st, ctypes.byref(table.native_optimizer), n, 1, bags, _POOLING[pooling],
                None if w is None else w.data_ptr(), g.data_ptr(), _GRAD_TRANSPORT[g.dtype],
                1 if validate_values else 0, None if flag is None else flag.data_ptr(), int(normalization_steps),
                None, inverse.data_ptr(), ws.data_ptr(), nbytes, stream,
            )
            order.give(inverse, first)
        if flag is not None:
            _raise_if_nonfinite(flag, self.stream)
        if not return_dedup:
            return None
        self.stream.synchronize()  # the unique count is read on the host
        u = int(count.item())
        first = first[:u]
        unique_keys = k[first] if u else k[:0]
        return unique_keys, inverse[:n], first



# ----------------------------------------------------------------------------
# PooledTableShard: the fused forward / backward hot path over T tables
# ----------------------------------------------------------------------------
class PooledTableShard:
    """T tables of one worker packed as ``[sum(rows), dim]`` in HBM.

    Bags are given in CSR form, table-major: for table ``t`` and sample ``b``
    the bag is ``ids[offsets[t*B + b] : offsets[t*B + b + 1]]`` with
    table-local row ids.  Pooled rows (forward output and pooled gradient) are
    ``[B, T, D]`` with ``layout="sample_major"`` (one group of T features, as
    ``gather_pooled`` returns it for target widths ``(T, M)``) or ``[T, B, D]``
    with ``layout="table_major"`` (T single-feature groups, the ``[B, 1, D]``
    outputs of T ``gather_pooled`` calls one after the other).
    """

    def __init__(self, table_rows: Sequence[int], dim: int, *, value_dtype: str = "bfloat16",
                 optimizer: Any = None, initializer: Any = None, seed: int = 0,
                 device: Any = None, layout: str = "sample_major"):
        if not torch.cuda.is_available():
            raise RuntimeError("PooledTableShard requires a ROCm GPU")
        if layout not in _LAYOUTS:
            raise ValueError(f"layout must be one of {sorted(_LAYOUTS)}, got {layout!r}")
        _native.library()
        self.layout = layout
        self._layout_code = _LAYOUTS[layout]
        self.device = _device_of(device)
        self.table_rows = [int(r) for r in table_rows]
        self.num_tables = len(self.table_rows)
        self.dim = int(dim)
        self.stream = torch.cuda.Stream(device=self.device)
        base = np.zeros(self.num_tables + 1, dtype=np.int64)
        base[1:] = np.cumsum(self.table_rows)
        self.total_rows = int(base[-1])
        generator = torch.Generator(device=self.device)
        generator.manual_seed(int(seed))
        with torch.cuda.stream(self.stream):
            self.row_base = torch.from_numpy(base).to(self.device)
            self.state = _TableState(self.total_rows, self.dim, value_dtype,
                                     optimizer if optimizer is not None else RowWiseAdagrad(),
                                     initializer, generator, self.device)
        self._workspace = _Workspace(self.device)
        torch.cuda.current_stream(self.device).wait_stream(self.stream)  # table initialized

    @property
    def table(self) -> torch.Tensor:
        return self.state.table

    def pooled_shape(self, batch_size: int) -> tuple[int, int, int]:
        """Shape of the pooled rows (and pooled gradient) of a batch in this shard's layout."""
        if self.layout == "table_major":
            return (self.num_tables, int(batch_size), self.dim)
        return (int(batch_size), self.num_tables, self.dim)

    def _csr(self, ids: Any, offsets: Any, batch_size: int):
        ids_t = contiguous(to_device(ids, self.device).reshape(-1))
        if ids_t.dtype not in (torch.int32, torch.int64):
            ids_t = ids_t.to(torch.int64)
        off = contiguous(to_device(offsets, self.device).reshape(-1).to(torch.int64))
        if off.numel() != self.num_tables * batch_size + 1:
            raise ValueError(
                f"offsets must have num_tables * batch_size + 1 = "
                f"{self.num_tables * batch_size + 1} entries, got {off.numel()}"
            )
        return ids_t, off

    def _weights(self, pooling: str, per_sample_weights: Any, n: int):
        if pooling not in _POOLING:
            raise ValueError(f"pooling must be one of {sorted(_POOLING)}, got {pooling!r}")
        if pooling != "weighted":
            return None
        if per_sample_weights is None:
            raise ValueError("weighted pooling requires per_sample_weights")
        w = contiguous(to_device(per_sample_weights, self.device).reshape(-1).to(torch.float32))
        if w.numel() != n:
            raise ValueError("per_sample_weights must have one weight per id")
        return w

    def lookup_pooled(self, ids: Any, offsets: Any, batch_size: int, *, pooling: str = "sum",
                      per_sample_weights: Any = None, out: torch.Tensor | None = None) -> torch.Tensor:
        """Forward: pooled rows in the storage dtype, ``pooled_shape(batch_size)``."""
        with _Ordered(self.stream, self.device) as order:
            ids_t, off = self._csr(ids, offsets, batch_size)
            w = self._weights(pooling, per_sample_weights, ids_t.numel())
            order.hold(ids_t, off, w, out)
            if out is None:
                out = torch.empty(self.pooled_shape(batch_size), dtype=self.state.table.dtype,
                                  device=self.device)
            _native.call(
                "flare_gather_pooled_csr", self.state.table.data_ptr(),
                storage_code(self.state.table.dtype), self.total_rows, self.dim,
                ids_t.data_ptr(), _native.INT32 if ids_t.dtype == torch.int32 else _native.INT64,
                ids_t.numel(), off.data_ptr(), self.num_tables, batch_size,
                self.row_base.data_ptr(), _POOLING[pooling], self._layout_code,
                None if w is None else w.data_ptr(), out.data_ptr(), int(self.stream.cuda_stream),
            )
            order.give(out)
        return out

    def _backward(self, ids, offsets, batch_size, pooled_grad, pooling, per_sample_weights,
                  normalization_steps, optimizer_override, want_dedup, validate_values=False):
        if isinstance(normalization_steps, bool) or not isinstance(normalization_steps, int) or normalization_steps <= 0:
            raise ValueError("normalization_steps must be a positive integer")
        with _Ordered(self.stream, self.device) as order:
            ids_t, off = self._csr(ids, offsets, batch_size)
            n = int(ids_t.numel())
            w = self._weights(pooling, per_sample_weights, n)
            g = _transport_grad(to_device(pooled_grad, self.device))
            order.hold(ids_t, off, w, g)
            if g.numel() != batch_size * self.num_tables * self.dim:
                raise ValueError(f"pooled gradient must be {list(self.pooled_shape(batch_size))} "
                                 f"({self.layout} layout)")
            opt = optimizer_override if optimizer_override is not None else self.state.native_optimizer
            grad_out = None
            if opt.kind == _native.OPT_NONE:
                grad_out = torch.empty((max(n, 1), self.dim), dtype=torch.float32, device=self.device)
            unique = inverse = first = count = None
            if want_dedup or opt.kind == _native.OPT_NONE:
                unique = torch.empty(max(n, 1), dtype=torch.int64, device=self.device)
                inverse = torch.empty(max(n, 1), dtype=torch.int32, device=self.device)
                first = torch.empty(max(n, 1), dtype=torch.int64, device=self.device)
                count = torch.zeros(1, dtype=torch.int64, device=self.device)
            nbytes = _native.library().flare_pooled_backward_workspace_bytes(n, self.total_rows, self.dim)
            ws = self._workspace.get(nbytes)
            s0, s1, st = self.state.pointers()
            p = lambda t: None if t is None else t.data_ptr()  # noqa: E731
            flag = torch.empty(1, dtype=torch.int32, device=self.device) if validate_values else None
            stream = int(self.stream.cuda_stream)
            id_code = _native.INT32 if ids_t.dtype == torch.int32 else _native.INT64
            if g.dtype == torch.float32 and not validate_values:  # the one-call form
                _native.call(
                    "flare_pooled_backward", self.state.table.data_ptr(),
                    storage_code(self.state.table.dtype), self.total_rows, self.dim, s0, s1, st,
                    ctypes.byref(opt), ids_t.data_ptr(), id_code, n, off.data_ptr(),
                    self.num_tables, batch_size, self.row_base.data_ptr(), _POOLING[pooling], self._layout_code,
                    p(w), g.data_ptr(), int(normalization_steps), p(grad_out), p(unique), p(inverse),
                    p(first), p(count), ws.data_ptr(), nbytes, stream,
                )
            else:
                self._dedup_apply(ids_t, id_code, n, off, batch_size, pooling, w, g, opt, flag,
                                  normalization_steps, grad_out, unique, inverse, first, count, ws, nbytes)
            order.give(grad_out, unique, inverse, first, count)
        if flag is not None:
            _raise_if_nonfinite(flag, self.stream)
        if unique is None:
            return None
        self.stream.synchronize()  # the count is read on the host
        u = int(count.item())
        result = (unique[:u], inverse[:n], first[:u])
        if grad_out is not None:
            result = result + (grad_out[:u],)
        return result

    def _dedup_apply(self, ids_t, id_code, n, off, batch_size, pooling, w, g, opt, flag, normalization_steps,
                     grad_out, unique, inverse, first, count, ws, nbytes):
        p = lambda t: None if t is None else t.data_ptr()  # noqa: E731
        s0, s1, st = self.state.pointers()
        stream = int(self.stream.cuda_stream)
        _native.call(
            "flare_pooled_dedup", ids_t.data_ptr(), id_code, n, off.data_ptr(), self.num_tables, batch_size,
            self.row_base.data_ptr(), self.total_rows, self.dim, _POOLING[pooling], self._layout_code, p(unique),
            p(first),
            p(count), ws.data_ptr(), nbytes, stream,
        )
        _native.call(
            "flare_pooled_apply_ex", self.state.table.data_ptr(), storage_code(self.state.table.dtype),
            self.total_rows, self.dim, s0, s1, st, ctypes.byref(opt), n, self.num_tables, batch_size,
            _POOLING[pooling], p(w), g.data_ptr(), _GRAD_TRANSPORT[g.dtype], 0 if flag is None else 1, p(flag),
            int(normalization_steps), p(grad_out), p(inverse), ws.data_ptr(), nbytes, stream,
        )

    def apply_pooled_gradients(self, ids: Any, offsets: Any, batch_size: int, pooled_grad: Any, *,
                               pooling: str = "sum", per_sample_weights: Any = None,
                               normalization_steps: int = 1, return_dedup: bool = False,
                               validate_values: bool = False):
        """Backward + update: dedup, deterministic segment sum, optimizer on the rows.

        ``pooled_grad`` may be float32 or bfloat16 (the gradient transport dtypes; bfloat16 is
        widened on load).  With ``validate_values`` an inf / NaN gradient updates nothing and
        raises ``FloatingPointError`` (synchronizes).  With ``return_dedup`` also returns
        ``(unique_rows, inverse, first_indices)`` (global rows; synchronizes once to read the
        unique count).
        """
        return self._backward(ids, offsets, batch_size, pooled_grad, pooling, per_sample_weights,
                              normalization_steps, None, return_dedup, validate_values)

    def reduce_pooled_gradients(self, ids: Any, offsets: Any, batch_size: int, pooled_grad: Any, *,
                                pooling: str = "sum", per_sample_weights: Any = None):
        """Backward only: ``(unique_rows, inverse, first_indices, grads[U, D])``."""
        none = _native.FlareOptimizer()
        none.kind = _native.OPT_NONE
        return self._backward(ids, offsets, batch_size, pooled_grad, pooling, per_sample_weights,
                              1, none, True)

    def plan_step(self, ids: Any, offsets: Any, batch_size: int, *, pooling: str = "sum",
                  per_sample_weights: Any = None) -> "PooledStepPlan":
        """Bind one batch's device buffers for allocation-free forward / dedup / apply."""
        return PooledStepPlan(self, ids, offsets, batch_size, pooling, per_sample_weights)

    def synchronize(self) -> None:
        self.stream.synchronize()


class PooledStepPlan:
    """One batch of a ``PooledTableShard``, with every buffer allocated up front.

    ``forward()`` pools into ``self.pooled``; ``dedup()`` sorts the ids and
    writes ``unique`` / ``first_indices`` / ``unique_count`` (device);
    ``apply(pooled_grad)`` reduces the gradient, updates the rows and writes
    ``inverse``.  No call allocates or synchronizes, so a loop of steps stays
    asynchronous on the shard's stream.  Called with another stream current,
    each call first makes the shard's stream wait for it and then makes it wait
    for the shard's stream; under ``torch.cuda.stream(shard.stream)`` there is
    nothing to order.
    """

    def __init__(self, shard: PooledTableShard, ids: Any, offsets: Any, batch_size: int,
                 pooling: str, per_sample_weights: Any):
        self.shard = shard
        self.batch = int(batch_size)
        self.pooling = pooling
        dev = shard.device
        with torch.cuda.stream(shard.stream):
            self.ids, self.offsets = shard._csr(ids, offsets, self.batch)
            self.n = int(self.ids.numel())
            self.weights = shard._weights(pooling, per_sample_weights, self.n)
            self.pooled = torch.empty(shard.pooled_shape(self.batch), dtype=shard.state.table.dtype, device=dev)
            m = max(self.n, 1)
            self.unique = torch.empty(m, dtype=torch.int64, device=dev)
            self.first_indices = torch.empty(m, dtype=torch.int64, device=dev)
            self.inverse = torch.empty(m, dtype=torch.int32, device=dev)
            self.unique_count = torch.zeros(1, dtype=torch.int64, device=dev)
            self.nonfinite = torch.zeros(1, dtype=torch.int32, device=dev)
            self.workspace_bytes = _native.library().flare_pooled_backward_workspace_bytes(
                self.n, shard.total_rows, shard.dim)
            self.workspace = torch.empty(max(self.workspace_bytes, 1), dtype=torch.uint8, device=dev)
        self._id_code = _native.INT32 if self.ids.dtype == torch.int32 else _native.INT64
        self._stream = int(shard.stream.cuda_stream)
        self._dedup_stream: torch.cuda.Stream | None = None
        # one id per bag (offsets 0, 1, 2, ...) in table-major order: the dedup and the forward are
        # told, so that the dedup keeps no gradient row per occurrence and the forward reads each
        # bag's id with its offsets (both check the claim on the device)
        self._dedup_layout = shard._layout_code
        bags = self.batch * shard.num_tables
        if shard.layout == "table_major" and self.n == bags and bags > 0:
            with torch.cuda.stream(shard.stream):
                steps = torch.arange(bags + 1, dtype=self.offsets.dtype, device=dev)
                if bool(torch.equal(self.offsets, steps)):
                    self._dedup_layout |= _native.LAYOUT_ONE_ID_PER_BAG
        torch.cuda.current_stream(dev).wait_stream(shard.stream)

    def step(self, pooled_grad: torch.Tensor, normalization_steps: int = 1,
             grad_out: torch.Tensor | None = None, optimizer: Any = None) -> torch.Tensor:
        """Forward, dedup and apply of one training step, dedup overlapped with forward.

        (Over a stream of batches, ``PooledStepPipeline`` is faster: it overlaps each batch's
        dedup with the previous batch's update instead, where the two share the GPU better.)

        The dedup depends only on the ids, so it runs on a second stream (same
        default priority) while the forward pools rows on the shard's stream;
        the apply waits for both.  The dedup also waits for everything already
        queued on the shard's stream, so it never overwrites a workspace an
        earlier apply of this plan still reads.
        """
        main = self.shard.stream
        if self._dedup_stream is None:
            self._dedup_stream = torch.cuda.Stream(device=self.shard.device)
        aux = self._dedup_stream
        aux.wait_stream(main)
        self._dedup_on(int(aux.cuda_stream))
        done = torch.cuda.Event()
        done.record(aux)
        pooled = self.forward()
        main.wait_event(done)
        self.apply(pooled_grad, normalization_steps, grad_out, optimizer)
        return pooled

    def _enter(self) -> torch.cuda.Stream:
        """The caller's current stream, which the shard's stream now waits for."""
        caller = torch.cuda.current_stream(self.shard.device)
        if caller != self.shard.stream:
            self.shard.stream.wait_stream(caller)
        return caller

    def _leave(self, caller: torch.cuda.Stream) -> None:
        if caller != self.shard.stream:
            caller.wait_stream(self.shard.stream)

    def forward(self) -> torch.Tensor:
        s = self.shard
        caller = self._enter()
        _native.call(
            "flare_gather_pooled_csr", s.state.table.data_ptr(), storage_code(s.state.table.dtype),
            s.total_rows, s.dim, self.ids.data_ptr(), self._id_code, self.n, self.offsets.data_ptr(),
            s.num_tables, self.batch, s.row_base.data_ptr(), _POOLING[self.pooling], self._dedup_layout,
            None if self.weights is None else self.weights.data_ptr(), self.pooled.data_ptr(),
            self._stream,
        )
        self._leave(caller)
        return self.pooled

    def dedup(self) -> None:
        caller = self._enter()
        self._dedup_on(self._stream)
        self._leave(caller)

    def _dedup_on(self, stream: int) -> None:
        s = self.shard
        _native.call(
            "flare_pooled_dedup", self.ids.data_ptr(), self._id_code, self.n, self.offsets.data_ptr(),
            s.num_tables, self.batch, s.row_base.data_ptr(), s.total_rows, s.dim,
            _POOLING[self.pooling], self._dedup_layout, self.unique.data_ptr(), self.first_indices.data_ptr(),
            self.unique_count.data_ptr(), self.workspace.data_ptr(), self.workspace_bytes, stream,
        )

    def apply(self, pooled_grad: torch.Tensor, normalization_steps: int = 1,
              grad_out: torch.Tensor | None = None, optimizer: Any = None,
              validate_values: bool = False) -> None:
        """``pooled_grad``: contiguous float32 or bfloat16 ``[batch, num_tables, dim]`` on the
        shard's device.  ``validate_values`` checks it first: inf / NaN updates nothing and
        raises ``FloatingPointError`` (this synchronizes)."""
        s = self.shard
        if pooled_grad.dtype not in _GRAD_TRANSPORT or not pooled_grad.is_contiguous() or \
                pooled_grad.numel() != self.batch * s.num_tables * s.dim or pooled_grad.device != s.device:
            raise ValueError(f"pooled_grad must be a contiguous float32 or bfloat16 {list(s.pooled_shape(self.batch))} "
                             f"device tensor ({s.layout} layout)")
        opt = s.state.native_optimizer if optimizer is None else optimizer
        s0, s1, st = s.state.pointers()
        caller = self._enter()
        if caller != s.stream:
            pooled_grad.record_stream(s.stream)
            if grad_out is not None:
                grad_out.record_stream(s.stream)
        _native.call(
            "flare_pooled_apply_ex", s.state.table.data_ptr(), storage_code(s.state.table.dtype),
            s.total_rows, s.dim, s0, s1, st, ctypes.byref(opt), self.n, s.num_tables, self.batch,
            _POOLING[self.pooling], None if self.weights is None else self.weights.data_ptr(),
            pooled_grad.data_ptr(), _GRAD_TRANSPORT[pooled_grad.dtype], 1 if validate_values else 0,
            self.nonfinite.data_ptr() if validate_values else None, int(normalization_steps),
            None if grad_out is None else grad_out.data_ptr(), self.inverse.data_ptr(),
            self.workspace.data_ptr(), self.workspace_bytes, self._stream,
        )
        self._leave(caller)
        if validate_values:
            _raise_if_nonfinite(self.nonfinite, s.stream)


def _mark(marks: dict, key: str, stream: torch.cuda.Stream) -> None:
    """Record a timing event under ``key`` when the caller asked for that phase boundary."""
    if key in marks:
        ev = torch.cuda.Event(enable_timing=True)
        ev.record(stream)
        marks[key] = ev


class PooledStepPipeline:
    """Training steps over a ring of bound batches, each batch's dedup one step ahead.

    The dedup of a batch needs only its ids, as the reference's input worker computes the
    unique ids of a batch ahead of the step that consumes it
    (``src/flare/runtime/fluxway/workers/sparse_input.py:333-349``).  ``forward(i)`` pools
    batch ``i`` on the shard's stream and queues batch ``i + 1``'s dedup on a second stream
    (default priority), where it runs while the caller's dense network and batch ``i``'s update
    run; ``update(i, grad)`` waits for batch ``i``'s own dedup and applies the update.  Each
    plan has its own workspace, and a dedup starts only after everything queued before it on
    the shard's stream, so it never overwrites a workspace an earlier update still reads.
    Steps go in order ``0, 1, 2, ...``, each ``forward`` followed by its ``update``;
    ``finish()`` waits for the dedup still running ahead.
    """

    def __init__(self, plans: Sequence[PooledStepPlan]):
        if len(plans) < 2:
            raise ValueError("a pipeline needs at least 2 plans (the next batch's dedup runs beside "
                             "the current batch's update, each in its own workspace)")
        shards = {id(p.shard) for p in plans}
        if len(shards) != 1:
            raise ValueError("the plans of a pipeline must belong to one shard")
        self.plans = list(plans)
        self.shard = self.plans[0].shard
        self.stream = torch.cuda.Stream(device=self.shard.device)
        self._next = 0  # the step whose forward comes next
        self._pending: int | None = None  # the step whose update comes next
        self._ready: dict[int, torch.cuda.Event] = {}  # step -> its dedup, run ahead

    def _plan(self, i: int) -> PooledStepPlan:
        return self.plans[i % len(self.plans)]

    def forward(self, i: int, marks: dict | None = None) -> torch.Tensor:
        """Pool batch ``i`` (``plans[i % len(plans)]``) and queue batch ``i + 1``'s dedup.

        ``marks`` (optional, for timing): a dict whose keys name phase boundaries to record as
        timing events -- ``"forward_done"`` on the shard's stream, ``"dedup_start"`` /
        ``"dedup_done"`` (batch ``i + 1``'s dedup) on the pipeline's stream.
        """
        if i != self._next or self._pending is not None:
            raise ValueError(f"pipeline steps go in order, each forward followed by its update: "
                             f"expected forward {self._next}" if self._pending is None else
                             f"expected update {self._pending} before forward {i}")
        marks = {} if marks is None else marks
        p = self._plan(i)
        main = self.shard.stream
        caller = p._enter()
        if i not in self._ready:  # the first step: its dedup has not run ahead
            p._dedup_on(int(main.cuda_stream))
        pooled = p.forward()  # does not wait for a dedup still running ahead
        _mark(marks, "forward_done", main)
        # batch i+1's plan is free: its last update is queued on the shard's stream before here
        self.stream.wait_stream(main)
        _mark(marks, "dedup_start", self.stream)
        self._plan(i + 1)._dedup_on(int(self.stream.cuda_stream))
        ready = torch.cuda.Event(enable_timing="dedup_done" in marks)
        ready.record(self.stream)
        self._ready[i + 1] = ready
        if "dedup_done" in marks:
            marks["dedup_done"] = ready
        p._leave(caller)
        self._pending = i
        return pooled

    def update(self, i: int, pooled_grad: torch.Tensor, normalization_steps: int = 1,
               grad_out: torch.Tensor | None = None, optimizer: Any = None,
               marks: dict | None = None) -> None:
        """Batch ``i``'s update (``PooledStepPlan.apply``) once its dedup is done.  ``marks``:
        ``"update_start"`` / ``"update_done"`` on the shard's stream."""
        if self._pending != i:
            raise ValueError(f"update {i} without its forward (pending: {self._pending})")
        marks = {} if marks is None else marks
        p = self._plan(i)
        main = self.shard.stream
        caller = p._enter()
        ready = self._ready.pop(i, None)
        if ready is not None:
            main.wait_event(ready)
        _mark(marks, "update_start", main)
        p.apply(pooled_grad, normalization_steps, grad_out, optimizer)
        _mark(marks, "update_done", main)
        p._leave(caller)
        self._pending = None
        self._next = i + 1

    def step(self, i: int, pooled_grad: torch.Tensor, normalization_steps: int = 1,
             grad_out: torch.Tensor | None = None, optimizer: Any = None,
             marks: dict | None = None) -> torch.Tensor:
        """``forward(i)`` then ``update(i, pooled_grad)``: a step whose gradient is known up
        front (benchmarks, replays)."""
        pooled = self.forward(i, marks)
        self.update(i, pooled_grad, normalization_steps, grad_out, optimizer, marks)
        return pooled

    def finish(self) -> None:
        """Make the shard's stream (and the caller's) wait for the dedup still running ahead."""
        for ready in self._ready.values():
            self.shard.stream.wait_event(ready)
            torch.cuda.current_stream(self.shard.device).wait_event(ready)
