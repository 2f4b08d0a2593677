"""Seeded synthetic inputs for the five sparse-embedding workloads.

1. 1 table x 1e6 rows, dim 64 fp32, batch 4096, bags U[1,20], Zipf 1.05,
   sum pooling, row-wise Adagrad (lr 0.01, eps 1e-8), init U(-0.05, 0.05)
2. 26 tables, rows log-uniform in [1e3, 1e7], dim 128 bf16, batch 65536,
   one id per bag, Zipf 1.1, row-wise Adagrad
3. 8 tables x 5e6 rows, dim 64 fp16, batch 16384, bags geometric(mean 30)
   capped at 500, Zipf 1.05, per-sample weights U(0,1), weighted-sum and mean
   pooling, backward to reduced gradients
4. 26 tables x 2e6 rows, dim 128 bf16, batch 65536, bags U[1,8], Zipf 1.3,
   row-wise Adagrad (high duplication)
5. 1 table x 1e8 rows, dim 128 bf16, Adam with fp32 m/v, batch 131072,
   bags U[1,64], Zipf 1.05

Ids are bounded-Zipf ranks (``p(r) ~ (r+1)^-alpha`` over ``[0, R)``), sampled
by inverse CDF with an exact head and an integral tail, mapped to rows by the
bijection ``row = (r*A + C) mod R`` so hot rows are not contiguous.  Per-table
seed ``1000*config + t`` (plus ``100000*batch_index`` for rotated batches).
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

_PRIMES = (2654435761, 2246822519, 3266489917, 668265263, 374761393, 1000003, 999983)


@dataclass
class Workload:
    config: int
    table_rows: list[int]
    dim: int
    value_dtype: str
    batch: int
    pooling: str
    optimizer: str  # "rowwise_adagrad" | "adam" | "none"
    ids: np.ndarray  # int64, table-major CSR values (table-local rows)
    offsets: np.ndarray  # int64 [T*B + 1]
    weights: np.ndarray | None = None
    init_range: float = 0.01
    extra_pooling: tuple[str, ...] = field(default_factory=tuple)

    @property
    def num_tables(self) -> int:
        return len(self.table_rows)

    @property
    def num_ids(self) -> int:
        return int(self.ids.size)

    @property
    def total_rows(self) -> int:
        return int(sum(self.table_rows))

    def row_base(self) -> np.ndarray:
        base = np.zeros(self.num_tables + 1, dtype=np.int64)
        base[1:] = np.cumsum(self.table_rows)
        return base

    def global_keys(self) -> np.ndarray:
        lengths = np.diff(self.offsets)
        table_of = np.repeat(np.arange(self.num_tables * self.batch), lengths) // self.batch
        return self.row_base()[table_of] + self.ids


def bounded_zipf(rng: np.random.Generator, n: int, rows: int, alpha: float, head: int = 1 << 16) -> np.ndarray:
    """Ranks in ``[0, rows)`` with ``p(r) ~ (r+1)^-alpha``."""
    h = min(rows, head)
    x = np.arange(1, h + 1, dtype=np.float64)
    head_w = x ** (-alpha)
    head_cdf = np.cumsum(head_w)
    head_mass = head_cdf[-1]
    one = 1.0 - alpha
    if rows > h:
        lo = (h + 0.5) ** one
        hi = (rows + 0.5) ** one
        tail_mass = (hi - lo) / one
    else:
        lo = tail_mass = 0.0
    u = rng.random(n) * (head_mass + tail_mass)
    ranks = np.empty(n, dtype=np.int64)
    in_head = u < head_mass
    ranks[in_head] = np.searchsorted(head_cdf, u[in_head], side="right")
    if rows > h:
        t = u[~in_head] - head_mass
        xs = (lo + t * one) ** (1.0 / one)
        ranks[~in_head] = np.clip(np.rint(xs).astype(np.int64) - 1, h, rows - 1)
    return np.minimum(ranks, rows - 1)


def rank_to_row(ranks: np.ndarray, rows: int, seed: int) -> np.ndarray:
    a = next(p for p in _PRIMES if math.gcd(p, rows) == 1 and p % rows != 0) if rows > 1 else 1
    c = (seed * 7919) % max(rows, 1)
    return ((ranks % rows) * (a % rows) + c) % max(rows, 1)


def _bag_lengths(rng: np.random.Generator, config: int, batch: int) -> np.ndarray:
    if config == 1:
        return rng.integers(1, 21, batch)
    if config == 2:
        return np.ones(batch, dtype=np.int64)
    if config == 3:
        return np.minimum(rng.geometric(1.0 / 30.0, batch), 500)
    if config == 4:
        return rng.integers(1, 9, batch)
    if config == 5:
        return rng.integers(1, 65, batch)
    raise ValueError(f"unknown config {config}")


_ALPHA = {1: 1.05, 2: 1.1, 3: 1.05, 4: 1.3, 5: 1.05}


def config_tables(config: int, row_scale: float = 1.0) -> tuple[list[int], int, str]:
    if config == 1:
        rows, dim, dtype = [1_000_000], 64, "float32"
    elif config == 2:
        rng = np.random.default_rng(1000 * config + 999)
        rows = np.floor(np.exp(rng.uniform(math.log(1e3), math.log(1e7), 26))).astype(np.int64).tolist()
        dim, dtype = 128, "bfloat16"
    elif config == 3:
        rows, dim, dtype = [5_000_000] * 8, 64, "float16"
    elif config == 4:
        rows, dim, dtype = [2_000_000] * 26, 128, "bfloat16"
    elif config == 5:
        rows, dim, dtype = [100_000_000], 128, "bfloat16"
    else:
        raise ValueError(f"unknown config {config}")
    rows = [max(16, int(r * row_scale)) for r in rows]
    return rows, dim, dtype


def make_workload(config: int, *, batch: int | None = None, row_scale: float = 1.0,
                  batch_index: int = 0) -> Workload:
    """Generate the ids (and weights) of one batch of a configuration."""
    rows, dim, dtype = config_tables(config, row_scale)
    full_batch = {1: 4096, 2: 65536, 3: 16384, 4: 65536, 5: 131072}[config]
    b = full_batch if batch is None else int(batch)
    ids_parts, len_parts = [], []
    for t, r in enumerate(rows):
        seed = 1000 * config + t + 100000 * batch_index
        rng = np.random.default_rng(seed)
        lengths = _bag_lengths(rng, config, b).astype(np.int64)
        ranks = bounded_zipf(rng, int(lengths.sum()), r, _ALPHA[config])
        ids_parts.append(rank_to_row(ranks, r, seed))
        len_parts.append(lengths)
    lengths = np.concatenate(len_parts)
    offsets = np.zeros(lengths.size + 1, dtype=np.int64)
    offsets[1:] = np.cumsum(lengths)
    ids = np.concatenate(ids_parts).astype(np.int64)
    weights = None
    pooling = "sum"
    optimizer = {1: "rowwise_adagrad", 2: "rowwise_adagrad", 3: "none", 4: "rowwise_adagrad", 5: "adam"}[config]
    extra = ()
    if config == 3:
        wrng = np.random.default_rng(1000 * config + 777 + 100000 * batch_index)
        weights = wrng.random(ids.size, dtype=np.float32)
        pooling = "weighted"
        extra = ("mean",)
    return Workload(config, rows, dim, dtype, b, pooling, optimizer, ids, offsets, weights,
                    0.05 if config == 1 else 0.01, extra)


def pooled_grad_host(workload: Workload, seed: int = 0) -> np.ndarray:
    """fp32 N(0, 1e-3) pooled gradients ``[B, T, D]`` (host; small sizes)."""
    rng = np.random.default_rng(1000 * workload.config + 555 + seed)
    return (rng.standard_normal((workload.batch, workload.num_tables, workload.dim), dtype=np.float32)
            * np.float32(1e-3)).astype(np.float32)
