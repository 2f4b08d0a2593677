"""HIP sparse-embedding operator: drop-in for ``CupySparseEmbeddingOperator``.

Mirrors ``src/flare/kernels/backends/gpu_cupy.py:23-556``: one stream per
operator instance (``:253``), conversions and launches for a call inside that
stream's context in the order convert -> reshape -> cast -> alloc -> launch
(``tests/kernels/test_sparse_embedding_backend.py:313-350``), empty inputs
return correctly shaped outputs without a launch (``:236-280``), and the pool
reclaimer runs when ``execution_context`` exits (``gpu_cupy.py:526-537``).

The kernels are hand-written HIP for gfx950 (``flare_amd/csrc``), reached
through the C ABI in ``include/flare_amd.h``.  Results are ``DeviceArray``s,
the CuPy array protocol the reference's callers use (numpy dtypes, ``astype``,
``__cuda_array_interface__``, DLPack).  Extensions over the reference:
bfloat16 storage, and ``pooling="mean" | "weighted"`` for ``gather_pooled``.
"""

from __future__ import annotations

import contextlib
from contextlib import AbstractContextManager
from typing import Any, Protocol

import torch

from flare_amd import _native
from flare_amd.array import DeviceArray
from flare_amd.contracts import SparseEmbeddingOperator, SparsePooledWidths, pooled_sparse_widths
from flare_amd.conversion import contiguous, storage_code, to_device

_POOLING = {"sum": _native.POOL_SUM, "mean": _native.POOL_MEAN, "weighted": _native.POOL_WEIGHTED}


class PoolReclaimer(Protocol):
    def after_operation(self, torch_module: Any) -> None: ...


class EagerPoolReclaimer:
    """Release cached device blocks after every operation (``cupy_memory.py:12-17``)."""

    def after_operation(self, torch_module: Any) -> None:
        torch_module.cuda.empty_cache()


class RetainPoolReclaimer:
    """Keep the allocator cache (``cupy_memory.py:20-24``)."""

    def after_operation(self, torch_module: Any) -> None:
        return None


class _OperatorStream:
    """The operator's stream as the reference exposes it: enter/exit and synchronize."""

    def __init__(self, stream: torch.cuda.Stream) -> None:
        self.torch_stream = stream
        self._ctx: list[Any] = []

    @property
    def ptr(self) -> int:
        return int(self.torch_stream.cuda_stream)

    def synchronize(self) -> None:
        self.torch_stream.synchronize()

    def __enter__(self):
        # inputs the caller is still producing on its own stream are complete
        # before this stream reads them
        caller = torch.cuda.current_stream(self.torch_stream.device)
        if caller != self.torch_stream:
            self.torch_stream.wait_stream(caller)
        ctx = torch.cuda.stream(self.torch_stream)
        ctx.__enter__()
        self._ctx.append(ctx)
        return self

    def __exit__(self, *exc) -> None:
        self._ctx.pop().__exit__(*exc)


class HipSparseEmbeddingOperator(SparseEmbeddingOperator):
    """Sparse gather / pooled gather / scatter on an MI355X through HIP kernels."""

    def __init__(
        self,
        value_dtype: str,
        gradient_dtype: str,
        empty_cache: bool = True,
        memory_reclaimer: PoolReclaimer | None = None,
        device: Any = None,
    ):
        super().__init__(value_dtype, gradient_dtype)
        if memory_reclaimer is not None and not callable(
            getattr(memory_reclaimer, "after_operation", None)
        ):
            raise TypeError("memory_reclaimer must implement after_operation")
        self.empty_cache = empty_cache
        self._memory_reclaimer = (
            memory_reclaimer
            if memory_reclaimer is not None
            else EagerPoolReclaimer() if empty_cache else RetainPoolReclaimer()
        )
        if not torch.cuda.is_available():
            raise RuntimeError("HipSparseEmbeddingOperator requires a ROCm GPU")
        _native.library()  # fail loudly now if the HIP library is missing
        self.device = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
        self.stream = _OperatorStream(torch.cuda.Stream(device=self.device))

    # ------------------------------------------------------------------ conversion
    def _array_on_stream(self, value: Any) -> torch.Tensor:
        tensor = to_device(value, self.device)
        if tensor.device.type == "cuda":
            tensor.record_stream(self.stream.torch_stream)
        return tensor

    def _inverse_on_stream(self, value: Any) -> torch.Tensor:
        tensor = self._array_on_stream(value)
        if tensor.dtype != torch.int32:
            tensor = tensor.to(torch.int32)
        return tensor

    def array(self, value: Any) -> DeviceArray:
        with self.stream:
            return DeviceArray(self._array_on_stream(value))

    def inverse(self, value: Any) -> DeviceArray:
        with self.stream:
            return DeviceArray(self._inverse_on_stream(value))

    def _workspace(self, nbytes: int) -> torch.Tensor:
        return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=self.device)

    # ------------------------------------------------------------------ forward
    def gather(self, emb_flat: Any, inverse: Any, batch_size: int, emb_dim: int,
               pad_index: int) -> DeviceArray:
        with self.stream:
            embedding = contiguous(self._array_on_stream(emb_flat).reshape(-1, emb_dim))
            inverse = contiguous(self._inverse_on_stream(inverse).reshape(-1))
            slots = int(inverse.numel())
            code = storage_code(embedding.dtype)
            if code is None:
                raise TypeError(
                    "sparse gather requires float16, bfloat16 or float32 embeddings, "
                    f"got {embedding.dtype}"
                )
            output = torch.empty((slots, emb_dim), dtype=embedding.dtype, device=self.device)
            if slots * emb_dim == 0:
                return DeviceArray(output.reshape(batch_size, 0, emb_dim))
            _native.call(
                "flare_gather", embedding.data_ptr(), code, embedding.shape[0], emb_dim,
                inverse.data_ptr(), slots, int(pad_index), output.data_ptr(), self.stream.ptr,
            )
            return DeviceArray(output.reshape(batch_size, -1, emb_dim))

    def gather_pooled(self, emb_flat: Any, inverse: Any, batch_size: int, emb_dim: int,
                      target_widths: SparsePooledWidths, pad_index: int, *,
                      pooling: str = "sum", per_sample_weights: Any = None) -> DeviceArray:
        with self.stream:
            feature_count, max_elements = pooled_sparse_widths(target_widths)
            embedding = contiguous(self._array_on_stream(emb_flat).reshape(-1, emb_dim))
            inverse = contiguous(self._inverse_on_stream(inverse).reshape(-1))
            code = storage_code(embedding.dtype)
            if code is None:
                raise TypeError(
                    "sparse pooled gather requires float16, bfloat16 or float32 embeddings, "
                    f"got {embedding.dtype}"
                )
            if pooling not in _POOLING:
                raise ValueError(f"pooling must be one of {sorted(_POOLING)}, got {pooling!r}")
            output = torch.empty((batch_size, feature_count, emb_dim), dtype=embedding.dtype,
                                 device=self.device)
            if batch_size * feature_count * emb_dim == 0:
                return DeviceArray(output)
            if inverse.numel() != batch_size * feature_count * max_elements:
                raise ValueError(
                    "pooled gather inverse slots must match batch_size * features * max_elements"
                )
            weights = None
            if pooling == "weighted":
                if per_sample_weights is None:
                    raise ValueError("weighted pooling requires per_sample_weights")
                weights = contiguous(self._array_on_stream(per_sample_weights).to(torch.float32).reshape(-1))
                if weights.numel() != inverse.numel():
                    raise ValueError("per_sample_weights must have one weight per inverse slot")
            _native.call(
                "flare_gather_pooled", embedding.data_ptr(), code, embedding.shape[0], emb_dim,
                inverse.data_ptr(), batch_size, feature_count, max_elements, int(pad_index),
                _POOLING[pooling], None if weights is None else weights.data_ptr(),
                output.data_ptr(), self.stream.ptr,
            )
            return DeviceArray(output)

    # ------------------------------------------------------------------ backward
    def _out_dtype(self, out_dtype: Any) -> torch.dtype:
        """Keyed-sum output dtype: the gradient dtype (float32), or the bfloat16 transport
        dtype, rounded as the sums are stored (the caller's grad.astype(transport),
        train_worker.py:518-522, fused into the scatter)."""
        if out_dtype is None:
            return torch.float32
        name = out_dtype if isinstance(out_dtype, str) else getattr(out_dtype, "name", str(out_dtype))
        if name in ("float32", "torch.float32"):
            return torch.float32
        if name in ("bfloat16", "torch.bfloat16"):
            return torch.bfloat16
        raise TypeError(f"scatter output dtype must be float32 or bfloat16, got {out_dtype!r}")

    def scatter(self, emb_rows: int, emb_dim: int, inverse: Any, pad_index: int,
                gradient: Any, *, out_dtype: Any = None) -> DeviceArray:
        with self.stream:
            inverse = contiguous(self._inverse_on_stream(inverse).reshape(-1))
            gradient = contiguous(
                self._array_on_stream(gradient).to(torch.float32).reshape(-1, emb_dim)
            )
            out_t = self._out_dtype(out_dtype)
            output = torch.empty((emb_rows, emb_dim), dtype=out_t, device=self.device)
            slots = int(inverse.numel())
            if gradient.shape[0] != slots:
                raise ValueError("scatter gradient rows must match inverse slots")
            nbytes = _native.library().flare_scatter_workspace_bytes(slots, emb_rows, emb_dim)
            workspace = self._workspace(nbytes)
            _native.call(
                "flare_scatter_ex", emb_rows, emb_dim, inverse.data_ptr(), slots, int(pad_index),
                gradient.data_ptr(), output.data_ptr(), storage_code(out_t), workspace.data_ptr(), nbytes,
                self.stream.ptr,
            )
            return DeviceArray(output)

    def scatter_pooled(self, emb_rows: int, emb_dim: int, inverse: Any, pad_index: int,
                       gradient: Any, target_widths: SparsePooledWidths, *,
                       out_dtype: Any = None) -> DeviceArray:
        with self.stream:
            feature_count, max_elements = pooled_sparse_widths(target_widths)
            inverse = contiguous(self._inverse_on_stream(inverse).reshape(-1))
            gradient = contiguous(
                self._array_on_stream(gradient).to(torch.float32).reshape(-1, feature_count, emb_dim)
            )
            slots = int(inverse.numel())
            pooled_slots = int(gradient.numel() // emb_dim)
            if slots != pooled_slots * max_elements:
                raise ValueError(
                    "pooled scatter inverse slots must match gradient rows times max_elements"
                )
            out_t = self._out_dtype(out_dtype)
            output = torch.empty((emb_rows, emb_dim), dtype=out_t, device=self.device)
            nbytes = _native.library().flare_scatter_workspace_bytes(slots, emb_rows, emb_dim)
            workspace = self._workspace(nbytes)
            _native.call(
                "flare_scatter_pooled_ex", emb_rows, emb_dim, inverse.data_ptr(), slots,
                int(pad_index), gradient.data_ptr(), pooled_slots // feature_count, feature_count,
                max_elements, output.data_ptr(), storage_code(out_t), workspace.data_ptr(), nbytes,
                self.stream.ptr,
            )
            return DeviceArray(output)

    # ------------------------------------------------------------------ lifecycle
    def execution_context(self) -> AbstractContextManager[Any]:
        @contextlib.contextmanager
        def _context():
            with self.stream:
                try:
                    yield self.stream
                finally:
                    self._memory_reclaimer.after_operation(torch)

        return _context()

    def prewarm(self) -> None:
        with self.execution_context():
            embedding = torch.arange(12, dtype=torch.float32, device=self.device).reshape(4, 3)
            inverse = torch.tensor([0, 4, 2, 1], dtype=torch.int32, device=self.device)
            gathered = self.gather(embedding, inverse, 4, 3, 4)
            scattered = self.scatter(
                4, 3, inverse, 4, torch.ones((4, 3), dtype=torch.float32, device=self.device)
            )
        self.stream.synchronize()
        if tuple(gathered.shape) != (4, 1, 3) or tuple(scattered.shape) != (4, 3):
            raise RuntimeError(
                "HIP sparse embedding kernel backend prewarm produced invalid shapes: "
                f"gather={tuple(gathered.shape)}, scatter={tuple(scattered.shape)}."
            )

    def take_device_errors(self) -> int:
        """Synchronize and return (then clear) the kernels' error bits."""
        return int(_native.library().flare_take_device_errors(self.stream.ptr))
