"""ctypes wrapper of ``oracle/_build/libcpu_step.so`` (the C restatement).

TEST INFRASTRUCTURE ONLY: used by tests and by ``bench.py``'s cpu_baseline
leg.  Storage arrays are numpy ``float32`` / ``float16`` or ``uint16`` bits for
bfloat16.
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "_build" / "libcpu_step.so"
ST = {"float32": 0, "float16": 1, "bfloat16": 2}
POOL = {"sum": 0, "mean": 1, "weighted": 2}
OPT = {"none": 0, "sgd": 1, "adam": 2, "rowwise_adagrad": 3}

_lib = None


def library():
    global _lib
    if _lib is None:
        if not LIB.exists():
            subprocess.run(["make", "-C", str(HERE)], check=True, capture_output=True)
        lib = ctypes.CDLL(str(LIB))
        vp, i32, i64, f32, f64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_float, ctypes.c_double
        lib.cpu_threads.restype = ctypes.c_int
        lib.cpu_set_threads.argtypes = [ctypes.c_int]
        lib.cpu_now.restype = f64
        lib.cpu_init_table.argtypes = [vp, ctypes.c_int, i64, f32, f32, ctypes.c_uint64]
        lib.cpu_pooled_forward.argtypes = [vp, ctypes.c_int, i32, vp, vp, i32, i64, vp, i32, vp, vp]
        lib.cpu_pooled_backward.restype = i64
        lib.cpu_pooled_backward.argtypes = [vp, ctypes.c_int, i32, vp, vp, vp, i32, f64, f64, f64, f64,
                                            vp, vp, i32, i64, vp, i32, vp, vp, vp, vp, vp]
        _lib = lib
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data


def threads() -> int:
    return int(library().cpu_threads())


def set_threads(n: int) -> None:
    """OpenMP threads of the following calls (the host's count by default)."""
    library().cpu_set_threads(int(n))


def init_table(rows: int, dim: int, storage: str, lo: float, hi: float, seed: int) -> np.ndarray:
    dtype = {"float32": np.float32, "float16": np.float16, "bfloat16": np.uint16}[storage]
    table = np.empty((rows, dim), dtype=dtype)
    library().cpu_init_table(_p(table), ST[storage], table.size, lo, hi, seed)
    return table


def pooled_forward(table, storage, dim, ids, offsets, num_tables, batch, row_base, pooling="sum", weights=None):
    out = np.empty((batch, num_tables, dim), dtype=table.dtype)
    ids = np.ascontiguousarray(ids, dtype=np.int64)
    offsets = np.ascontiguousarray(offsets, dtype=np.int64)
    row_base = np.ascontiguousarray(row_base, dtype=np.int64)
    w = None if weights is None else np.ascontiguousarray(weights, dtype=np.float32)
    library().cpu_pooled_forward(_p(table), ST[storage], dim, _p(ids), _p(offsets), num_tables, batch,
                                 _p(row_base), POOL[pooling], _p(w), _p(out))
    return out


def pooled_backward(table, storage, dim, state, optimizer, ids, offsets, num_tables, batch, row_base,
                    pooled_grad, pooling="sum", weights=None, lr=0.01, beta1=0.9, beta2=0.999, eps=1e-8):
    """In place on ``table`` / ``state``.  Returns (unique, inverse, grads) per table-local dedup."""
    ids = np.ascontiguousarray(ids, dtype=np.int64)
    offsets = np.ascontiguousarray(offsets, dtype=np.int64)
    row_base = np.ascontiguousarray(row_base, dtype=np.int64)
    g = np.ascontiguousarray(pooled_grad, dtype=np.float32)
    w = None if weights is None else np.ascontiguousarray(weights, dtype=np.float32)
    n = ids.size
    unique = np.empty(max(n, 1), np.int64)
    inverse = np.empty(max(n, 1), np.int32)
    grad_out = np.empty((max(n, 1), dim), np.float32) if optimizer == "none" else None
    s0 = state.get("acc", state.get("m"))
    s1 = state.get("v")
    st = state.get("step")
    u = library().cpu_pooled_backward(
        _p(table), ST[storage], dim, _p(s0), _p(s1), _p(st), OPT[optimizer], lr, beta1, beta2, eps,
        _p(ids), _p(offsets), num_tables, batch, _p(row_base), POOL[pooling], _p(w), _p(g),
        _p(grad_out), _p(unique), _p(inverse))
    return int(u), unique, inverse, grad_out


def now() -> float:
    return float(library().cpu_now())
