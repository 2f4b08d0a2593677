"""CPU oracle for Flare's sparse-embedding hot path (numpy restatement).

TEST INFRASTRUCTURE ONLY.  This module restates the reference's algorithms so
that tests can check the HIP path against them; it is never imported by the
product package ``flare_amd``.

Storage dtypes are numpy ``float32`` / ``float16``; bfloat16 (absent from
numpy) is carried as ``uint16`` bit patterns and converted with
round-to-nearest-even from the IEEE-754 definition.

Every public function names the reference lines it follows.  Where the
reference has no definition (bf16 storage, mean / weighted pooling, row-wise
Adagrad, the deterministic reduction order) the docstring says so and states
the closed form used instead.

How each part is pinned (tests/test_oracle.py, tests/test_golden.py):

* unique_first_occurrence_*: the reference's literal vectors
  (tests/runtime/test_sparse_input_resources.py:77-123) and a dict brute force.
* gather / gather_pooled (sum): the reference's known answers
  (tests/kernels/test_sparse_embedding_backend.py:78-89,144-183,225-233) and
  the audit restatement padded[inverse].sum(axis=2).
* mean / weighted pooling, gather_pooled_csr: closed forms and the CSR ==
  materialized-padded identity.
* bf16 rounding: torch.bfloat16 casts.
* scatter / scatter_pooled / segment_sums: the reference's own test cases and
  np.add.at; one-unit keys equal the plain slot-order sum bit for bit.
* adam_update: the reference's two-step known answer and a float64 textbook.
* rowwise_adagrad_update: the optax closed form it reduces to at D == 1 and
  the row mean of squares.
* sgd_update: the flush-window known answer.
* nested_global_positions: the reference's vector (test_sparse_input_resources.py:77-105) and
  a brute force that lays ragged batches out densely.
* KeyMap (the dynamic store's key -> row map): a dict restatement of
  first-occurrence row assignment, checked by closed-form sequences and
  invariants; its mixing function splitmix64 by the published SplitMix64
  outputs for seed 1234567; keymap_initial_values by its range, moments and
  independence from the batch.  The initial values themselves have no
  counterpart in the reference (its store's initializer stream is external):
  parity unpinned against the reference, pinned only as this library's own
  definition.

Parity unpinned (only the external sparse_embedding store defines these, and
it is not available here): the rounding of updated fp16 / bf16 rows (RNE is
used), and the division of the summed gradient by normalization_steps for
Adam and row-wise Adagrad (pinned only for SGD by the flush-window test).
"""

from __future__ import annotations

import math

import numpy as np

# --------------------------------------------------------------------------
# dtype helpers (IEEE-754 definitions; no library rounding code is reused)
# --------------------------------------------------------------------------


def f32_to_bf16_bits(values: np.ndarray) -> np.ndarray:
    """Round float32 to bfloat16 (nearest, ties to even); returns uint16 bits.

    NaN keeps a quiet NaN payload; infinities and overflow follow IEEE rules
    (overflow rounds to +-inf).
    """
    f = np.ascontiguousarray(values, dtype=np.float32)
    bits = f.view(np.uint32).astype(np.uint64)
    lsb = (bits >> np.uint64(16)) & np.uint64(1)
    rounded = (bits + np.uint64(0x7FFF) + lsb) >> np.uint64(16)
    nan = np.isnan(f)
    out = rounded.astype(np.uint16)
    out[nan] = ((bits[nan] >> np.uint64(16)) | np.uint64(0x40)).astype(np.uint16)
    return out


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(bits, dtype=np.uint16).astype(np.uint32) << np.uint32(16)
    return b.view(np.float32)


STORAGE_DTYPES = ("float32", "float16", "bfloat16")


def storage_to_f32(values: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "bfloat16":
        return bf16_bits_to_f32(values)
    return np.asarray(values).astype(np.float32)


def f32_to_storage(values: np.ndarray, dtype: str) -> np.ndarray:
    """fp32 -> storage dtype with round-to-nearest-even (numpy's fp16 cast is RNE)."""
    if dtype == "bfloat16":
        return f32_to_bf16_bits(values)
    if dtype == "float16":
        return np.asarray(values, dtype=np.float32).astype(np.float16)
    return np.asarray(values, dtype=np.float32).copy()


# --------------------------------------------------------------------------
# a7: pooled_sparse_widths  (src/flare/ops/contracts.py:7-19)
# --------------------------------------------------------------------------


def pooled_sparse_widths(target_widths) -> tuple[int, int]:
    """Follows ``src/flare/ops/contracts.py:7-19``: exactly two positive widths."""
    if len(target_widths) != 2:
        raise ValueError("exactly two target widths required")
    f, m = (int(v) for v in target_widths)
    if f <= 0 or m <= 0:
        raise ValueError("positive target widths required")
    return f, m


# --------------------------------------------------------------------------
# a1: unique_first_occurrence  (src/flare/ops/sparse_unique.py:13-77)
# --------------------------------------------------------------------------

_HASH_MULTIPLIER = 11400714819323198485
_U64 = (1 << 64) - 1


def unique_first_occurrence_hash(values: np.ndarray):
    """Serial open-addressing dedup, as ``sparse_unique.py:24-48`` does it.

    Capacity is the smallest power of two with ``2*cap >= 3*N``; the probe
    start is ``(u64(key) * 11400714819323198485) & mask`` with linear probing.
    Returns ``(unique, inverse:int32, first_indices:int64)`` in first-occurrence
    order.  Empty input returns ``(values.copy(), int32[0], int64[0])``
    (``sparse_unique.py:61-66``); non-integer keys raise TypeError
    (``:59-60``).  Pure-Python loop: small inputs only.
    """
    values = np.asarray(values)
    if values.ndim != 1:
        values = values.reshape(-1)
    if values.dtype.kind not in "iu":
        raise TypeError(f"sparse unique requires integer keys, got {values.dtype}")
    n = values.size
    if n == 0:
        return values.copy(), np.empty(0, np.int32), np.empty(0, np.int64)
    capacity = 1
    while capacity * 2 < n * 3:
        capacity <<= 1
    mask = capacity - 1
    keys = [None] * capacity
    ids = [0] * capacity
    unique, first, inverse = [], [], np.empty(n, np.int32)
    for index, key in enumerate(values.tolist()):
        slot = ((key & _U64) * _HASH_MULTIPLIER & _U64) & mask
        while keys[slot] is not None and keys[slot] != key:
            slot = (slot + 1) & mask
        if keys[slot] is None:
            keys[slot] = key
            ids[slot] = len(unique)
            inverse[index] = len(unique)
            unique.append(key)
            first.append(index)
        else:
            inverse[index] = ids[slot]
    return (
        np.asarray(unique, dtype=values.dtype),
        inverse,
        np.asarray(first, dtype=np.int64),
    )


def unique_first_occurrence_sorted(values: np.ndarray):
    """Sort-based dedup re-ordered to first occurrence (``sparse_input.py:150-163``).

    ``np.unique(return_index, return_inverse)`` then ``argsort(first_indices)``
    and an inverse remap, as the reference's GPU branch does with CuPy.  A
    second, independent formulation of ``unique_first_occurrence_hash``.
    """
    values = np.asarray(values).reshape(-1)
    if values.dtype.kind not in "iu":
        raise TypeError(f"sparse unique requires integer keys, got {values.dtype}")
    if values.size == 0:
        return values.copy(), np.empty(0, np.int32), np.empty(0, np.int64)
    unique, first, inverse = np.unique(values, return_index=True, return_inverse=True)
    order = np.argsort(first, kind="stable")
    remap = np.empty(order.size, dtype=np.int32)
    remap[order] = np.arange(order.size, dtype=np.int32)
    return unique[order], remap[inverse.reshape(-1)], first[order].astype(np.int64)


# --------------------------------------------------------------------------
# a3: gather  (src/flare/kernels/backends/gpu_cupy.py:52-73,108-132,332-371;
#              src/flare/ops/sparse_gather.py:15-36)
# --------------------------------------------------------------------------


def gather(emb: np.ndarray, inverse: np.ndarray, batch_size: int, dim: int, pad_index: int):
    """``out[slot] = emb[inv[slot]]`` or 0 where ``inv == pad_index``.

    Output keeps the storage dtype (bf16 as uint16 bits) and shape
    ``[batch_size, slots // batch_size, dim]`` (``gpu_cupy.py:371``).
    """
    emb2 = np.asarray(emb).reshape(-1, dim)
    inv = np.asarray(inverse).reshape(-1).astype(np.int64)
    out = np.zeros((inv.size, dim), dtype=emb2.dtype)
    valid = inv != pad_index
    out[valid] = emb2[inv[valid]]
    if inv.size == 0:
        return out.reshape(batch_size, 0, dim)
    return out.reshape(batch_size, -1, dim)


# --------------------------------------------------------------------------
# a4: gather_pooled, padded [B, F, M] inverse
#     (gpu_cupy.py:74-107 fp32, :133-167 fp16; sparse_gather.py:39-148)
# --------------------------------------------------------------------------

POOLING_SUM, POOLING_MEAN, POOLING_WEIGHTED = "sum", "mean", "weighted"


def gather_pooled(
    emb: np.ndarray,
    inverse: np.ndarray,
    batch_size: int,
    dim: int,
    target_widths,
    pad_index: int,
    *,
    storage: str = "float32",
    pooling: str = POOLING_SUM,
    weights: np.ndarray | None = None,
):
    """Pooled gather with fp32 accumulation, summed sequentially in ``m``.

    ``out[b,f,:] = sum_{m<M, inv[b,f,m] != pad} emb[inv[b,f,m], :]`` with one
    fp32 accumulator per element (``gpu_cupy.py:96-103,156-163``), then rounded
    to the storage dtype (RNE, ``gpu_cupy.py:163``).

    Extensions with no reference implementation (closed forms):
      * ``mean``: divide the fp32 sum by ``max(#valid, 1)``
        (divisor of ``src/flare/jax/layers/embedding.py:120-126``);
      * ``weighted``: ``sum_m w[b,f,m] * e`` with the product rounded to fp32
        before the add.
    """
    f_count, m_count = pooled_sparse_widths(target_widths)
    e32 = storage_to_f32(np.asarray(emb).reshape(-1, dim), storage)
    inv = np.asarray(inverse).reshape(batch_size, f_count, m_count).astype(np.int64)
    acc = np.zeros((batch_size, f_count, dim), dtype=np.float32)
    count = np.zeros((batch_size, f_count), dtype=np.int64)
    w = None
    if pooling == POOLING_WEIGHTED:
        w = np.asarray(weights, dtype=np.float32).reshape(batch_size, f_count, m_count)
    for m in range(m_count):
        rows = inv[:, :, m]
        valid = rows != pad_index
        if not valid.any():
            continue
        vals = np.zeros((batch_size, f_count, dim), dtype=np.float32)
        vals[valid] = e32[rows[valid]]
        if w is not None:
            vals = (vals * w[:, :, m, None]).astype(np.float32)
        acc = np.where(valid[..., None], (acc + vals).astype(np.float32), acc)
        count += valid
    if pooling == POOLING_MEAN:
        acc = (acc / np.maximum(count, 1)[..., None].astype(np.float32)).astype(np.float32)
    return f32_to_storage(acc, storage)


# --------------------------------------------------------------------------
# CSR (ragged) pooled gather over several tables -- the layout the north-star
# workloads use.  Equivalent to materialize_padded_inverse + gather_pooled
# (recipes/recsys/ranking/schema/input.py:23-123 then gpu_cupy.py:373-420).
# --------------------------------------------------------------------------


def gather_pooled_csr(
    table: np.ndarray,
    ids: np.ndarray,
    offsets: np.ndarray,
    row_base: np.ndarray,
    batch_size: int,
    dim: int,
    *,
    storage: str = "float32",
    pooling: str = POOLING_SUM,
    weights: np.ndarray | None = None,
):
    """Bags are ordered table-major: bag ``k = t*B + b``; output ``[B, T, D]``;
    ``row_base`` has ``T + 1`` entries (the last is the total row count).

    ``out[b,t] = sum_{i in [offsets[k], offsets[k+1])} w_i * table[row_base[t] + ids[i]]``,
    accumulated in fp32 sequentially in ``i``, rounded to storage with RNE.
    """
    num_tables = int(np.asarray(row_base).size) - 1
    e32 = storage_to_f32(np.asarray(table).reshape(-1, dim), storage)
    ids = np.asarray(ids, dtype=np.int64)
    offsets = np.asarray(offsets, dtype=np.int64)
    bags = num_tables * batch_size
    lengths = np.diff(offsets)
    bag_of = np.repeat(np.arange(bags), lengths)
    table_of = bag_of // batch_size
    rows = row_base[table_of] + ids
    acc = np.zeros((bags, dim), dtype=np.float32)
    pos = offsets[:-1].copy()
    w = None if weights is None else np.asarray(weights, dtype=np.float32)
    max_len = int(lengths.max()) if lengths.size else 0
    for p in range(max_len):
        active = np.nonzero(lengths > p)[0]
        i = pos[active] + p
        vals = e32[rows[i]]
        if pooling == POOLING_WEIGHTED:
            vals = (vals * w[i, None]).astype(np.float32)
        acc[active] = (acc[active] + vals).astype(np.float32)
    if pooling == POOLING_MEAN:
        acc = (acc / np.maximum(lengths, 1)[:, None].astype(np.float32)).astype(np.float32)
    out = acc.reshape(num_tables, batch_size, dim).transpose(1, 0, 2)
    return f32_to_storage(np.ascontiguousarray(out), storage)


def materialize_padded_inverse(flat_values, nested_splits, *, pad_index, batch_size, target_widths):
    """Nested ragged -> padded ``[B, *target_widths]`` int32 (``schema/input.py:90-123``).

    Each level's children are placed at ``parent * width + local`` and dropped
    when ``local >= width`` (truncation cannot spill into the next row).
    Invalid offsets raise ``ValueError("Invalid ragged inverse offsets ...")``.
    """
    flat = np.asarray(flat_values).reshape(-1)
    splits = [np.asarray(s, dtype=np.int64) for s in nested_splits]
    if len(splits) != len(target_widths) or splits[0].size != batch_size + 1:
        raise ValueError("Ragged inverse shape mismatch")
    out = np.full((batch_size, *target_widths), pad_index, dtype=np.int32)
    positions = np.arange(batch_size, dtype=np.int64)
    valid = np.ones(batch_size, dtype=bool)
    for level, (split, width) in enumerate(zip(splits, target_widths)):
        children = splits[level + 1].size - 1 if level + 1 < len(splits) else flat.size
        if (split.ndim != 1 or split.size != positions.size + 1 or split[0] != 0
                or split[-1] != children or np.any(split[1:] < split[:-1])):
            raise ValueError(f"Invalid ragged inverse offsets at level {level}")
        lengths = np.diff(split)
        parents = np.repeat(np.arange(positions.size), lengths)
        local = np.arange(children) - split[parents]
        valid = valid[parents] & (local < width)
        positions = positions[parents] * width + local
    out.reshape(-1)[positions[valid]] = flat[valid].astype(np.int32)
    return out


def materialize_padded_inverse_csr(ids, offsets, batch_size, max_elements, pad_index):
    """CSR bags -> padded ``[B, 1, M]`` int32 (``schema/input.py:23-123``, one level).

    Ids beyond width ``M`` are truncated (``tests/kernels/test_sparse_cpu_parallel.py:74-87``).
    """
    out = np.full((batch_size, 1, max_elements), pad_index, dtype=np.int32)
    offsets = np.asarray(offsets, dtype=np.int64)
    for b in range(batch_size):
        seg = ids[offsets[b] : offsets[b + 1]][:max_elements]
        out[b, 0, : seg.size] = seg
    return out


# --------------------------------------------------------------------------
# Deterministic segment reduction order shared with the HIP path.
#
# The reference sums duplicate-key gradients either sequentially in slot order
# (Numba, sparse_scatter.py:14-56) or with float atomics in no fixed order
# (CuPy K5-K7, gpu_cupy.py:168-252).  The HIP path sorts occurrences stably by
# key and reduces each key's occurrences in occurrence order, cut into fixed
# "units" of REDUCE_UNIT consecutive sorted positions: a key's occurrences are
# summed sequentially inside each unit, and the unit partials are then folded
# left to right; a key of more than FOLD_CHUNK unit partials folds each run of
# FOLD_CHUNK partials left to right, then the run results left to right (so a
# very hot key's fold is parallel).  A key whose occurrences fall in one unit
# is summed exactly in slot order, i.e. bit-identically to the Numba reference.
# --------------------------------------------------------------------------

REDUCE_UNIT = 64


def sorted_occurrences(keys: np.ndarray, valid: np.ndarray | None = None):
    """Stable sort of occurrence indices by key; invalid occurrences dropped."""
    keys = np.asarray(keys).reshape(-1)
    idx = np.arange(keys.size, dtype=np.int64)
    if valid is not None:
        idx = idx[np.asarray(valid).reshape(-1)]
    order = np.argsort(keys[idx], kind="stable")
    perm = idx[order]
    sk = keys[perm]
    if sk.size:
        heads = np.concatenate([[True], sk[1:] != sk[:-1]])
    else:
        heads = np.zeros(0, dtype=bool)
    starts = np.nonzero(heads)[0]
    return perm, sk, starts


FOLD_CHUNK = 64  # unit partials per first-level fold run of a very hot key


def _segment_pieces(starts: np.ndarray, ends: np.ndarray, unit: int):
    """Cut each segment [start, end) of sorted positions at multiples of ``unit``:
    (segment of each piece, first absolute position, length)."""
    piece_seg, piece_a, piece_len = [], [], []
    for s, (a, e) in enumerate(zip(starts.tolist(), ends.tolist())):
        cut = a
        while cut < e:
            nxt = min(e, (cut // unit + 1) * unit)
            piece_seg.append(s)
            piece_a.append(cut)
            piece_len.append(nxt - cut)
            cut = nxt
    return np.asarray(piece_seg, np.int64), np.asarray(piece_a, np.int64), np.asarray(piece_len, np.int64)


def _segment_sums_by_pieces(rows_at, starts: np.ndarray, ends: np.ndarray, dim: int, unit: int) -> np.ndarray:
    """Sums of the segments [starts, ends) (absolute sorted positions), HIP order:
    sequential fp32 sums inside each (segment, unit) piece, then the pieces of each
    segment folded left to right (a segment of more than FOLD_CHUNK pieces: each run
    of FOLD_CHUNK pieces left to right, then the run results left to right).
    ``rows_at(positions)`` returns the contribution rows at absolute positions."""
    nseg = starts.size
    out = np.zeros((nseg, dim), dtype=np.float32)
    piece_seg, pa, plen = _segment_pieces(starts, ends, unit)
    if piece_seg.size == 0:
        return out
    partial = np.zeros((pa.size, dim), dtype=np.float32)
    for step in range(int(plen.max())):
        act = np.nonzero(plen > step)[0]
        partial[act] = (partial[act] + np.asarray(rows_at(pa[act] + step), np.float32)).astype(np.float32)
    first_piece = np.ones(pa.size, dtype=bool)
    first_piece[1:] = piece_seg[1:] != piece_seg[:-1]
    out[piece_seg[first_piece]] = partial[first_piece]
    heads = np.nonzero(first_piece)[0]
    counts = np.diff(np.append(heads, pa.size))
    for s0, c in zip(heads[counts > 1].tolist(), counts[counts > 1].tolist()):  # keys crossing units
        seg = piece_seg[s0]
        if c <= FOLD_CHUNK:
            acc = partial[s0].copy()
            for q in range(s0 + 1, s0 + c):
                acc = (acc + partial[q]).astype(np.float32)
        else:
            acc = None
            for c0 in range(0, c, FOLD_CHUNK):
                run = partial[s0 + c0].copy()
                for q in range(s0 + c0 + 1, s0 + min(c0 + FOLD_CHUNK, c)):
                    run = (run + partial[q]).astype(np.float32)
                acc = run if acc is None else (acc + run).astype(np.float32)
        out[seg] = acc
    return out


def segment_sums(contrib: np.ndarray, starts: np.ndarray, total: int, unit: int = REDUCE_UNIT):
    """Sum rows of ``contrib`` (already in sorted order) per segment, HIP order.

    ``starts`` are segment heads in sorted positions; ``total`` = #positions.
    Returns ``[len(starts), D]`` float32.
    """
    contrib = np.asarray(contrib, dtype=np.float32)
    dim = contrib.shape[1] if contrib.ndim == 2 else 0
    starts = np.asarray(starts, np.int64)
    ends = np.append(starts[1:], total).astype(np.int64)
    return _segment_sums_by_pieces(lambda pos: contrib[pos], starts, ends, dim, unit)


def segment_sums_selected(rows_at, starts: np.ndarray, ends: np.ndarray, dim: int, unit: int = REDUCE_UNIT):
    """``segment_sums`` of some segments only, each given by its absolute sorted positions
    ``[starts[i], ends[i])`` within the whole sorted occurrence stream (the unit cuts depend
    on those absolute positions); ``rows_at(positions)`` returns their contribution rows.
    For checking a sample of keys of a step too large to sum in full on the host."""
    return _segment_sums_by_pieces(rows_at, np.asarray(starts, np.int64), np.asarray(ends, np.int64), dim, unit)


def sequential_segment_sums(contrib: np.ndarray, starts: np.ndarray, total: int):
    """Plain slot-order fp32 sums (the Numba reference order, sparse_scatter.py:14-32)."""
    return segment_sums(contrib, starts, total, unit=max(total, 1))


# --------------------------------------------------------------------------
# a5 / a6: scatter and scatter_pooled (gpu_cupy.py:422-524; sparse_scatter.py:14-144)
# --------------------------------------------------------------------------


def scatter(emb_rows, dim, inverse, pad_index, gradient, *, unit=REDUCE_UNIT):
    """``out[r] = sum_{slot: inv[slot]=r} grad[slot]`` in fp32 ``[emb_rows, dim]``.

    Slots equal to ``pad_index`` (or outside ``[0, emb_rows)``) contribute nothing.
    """
    inv = np.asarray(inverse).reshape(-1).astype(np.int64)
    grad = np.asarray(gradient, dtype=np.float32).reshape(-1, dim)
    return _keyed_sum(emb_rows, dim, inv, pad_index, lambda slots: grad[slots], unit)


def scatter_pooled(emb_rows, dim, inverse, pad_index, gradient, target_widths, *, unit=REDUCE_UNIT):
    """Backward of sum pooling: each slot receives its bag's gradient row.

    Raises ValueError when ``slots != B*F*M`` (``gpu_cupy.py:479-483``).
    """
    f_count, m_count = pooled_sparse_widths(target_widths)
    inv = np.asarray(inverse).reshape(-1).astype(np.int64)
    grad = np.asarray(gradient, dtype=np.float32).reshape(-1, f_count, dim).reshape(-1, dim)
    if inv.size != grad.shape[0] * m_count:
        raise ValueError(
            "pooled scatter inverse slots must match gradient rows times max_elements"
        )
    return _keyed_sum(emb_rows, dim, inv, pad_index, lambda slots: grad[slots // m_count], unit)


def _keyed_sum(emb_rows, dim, inv, pad_index, rows_for, unit):
    out = np.zeros((emb_rows, dim), dtype=np.float32)
    valid = (inv != pad_index) & (inv >= 0) & (inv < emb_rows)
    perm, sk, starts = sorted_occurrences(inv, valid)
    if perm.size == 0:
        return out
    sums = segment_sums(rows_for(perm), starts, perm.size, unit)
    out[sk[starts]] = sums
    return out


# --------------------------------------------------------------------------
# a11 / a12 / a13: sparse optimizers on the deduplicated, summed gradient.
# --------------------------------------------------------------------------


def adam_update(w, m, v, step, g, *, lr=0.01, beta1=0.9, beta2=0.999, eps=1e-8):
    """Per-key Adam as restated in ``tools/validation/audit_sparse_training.py:460-471``.

    ``step += 1; m = b1*m + (1-b1)*g; v = b2*v + (1-b2)*g^2;
    w -= lr * (m / (1-b1^step)) / (sqrt(v / (1-b2^step)) + eps)``, fp32 state,
    bias corrections computed in double and rounded to fp32.
    Known answer pinned in tests: zero init, lr 0.1, grad 1 -> -0.1 then -0.2
    (``tests/runtime/test_sparse_storage_limits.py:41-119``).
    """
    f = np.float32
    step = np.asarray(step, dtype=np.int64) + 1
    g = np.asarray(g, dtype=f)
    m = (f(beta1) * m + f(1.0 - beta1) * g).astype(f)
    v = (f(beta2) * v + f(1.0 - beta2) * np.square(g)).astype(f)
    bc1 = (1.0 - np.power(float(beta1), step.astype(np.float64))).astype(f)
    bc2 = (1.0 - np.power(float(beta2), step.astype(np.float64))).astype(f)
    m_hat = (m / bc1[:, None]).astype(f)
    v_hat = (v / bc2[:, None]).astype(f)
    w = (w - f(lr) * m_hat / (np.sqrt(v_hat) + f(eps))).astype(f)
    return w, m, v, step.astype(np.int32)


def rowwise_adagrad_update(w, acc, g, *, lr=0.01, eps=1e-8):
    """Row-wise Adagrad (no reference implementation; closed form, FBGEMM style).

    One fp32 accumulator per row: ``acc += mean_d(g^2)``;
    ``w -= lr * g / (sqrt(acc) + eps)``.  Initial accumulator 0.  The
    elementwise optax form it reduces to for ``D == 1`` is pinned by
    ``tests/training/test_optimizer_factories.py:43-51``.
    """
    f = np.float32
    g = np.asarray(g, dtype=f)
    acc = (acc + np.mean(np.square(g.astype(np.float64)), axis=1)).astype(f)
    w = (w - f(lr) * g / (np.sqrt(acc)[:, None] + f(eps))).astype(f)
    return w, acc


def sgd_update(w, g, *, lr=0.01):
    """``w -= lr * g`` (``se.Sgd``; flush-window behaviour, test_checkpointing.py:229-251)."""
    f = np.float32
    return (w - f(lr) * np.asarray(g, dtype=f)).astype(f)


# --------------------------------------------------------------------------
# Fused sparse step on a dense row-indexed table shard:
#   forward  : CSR pooled gather                      (a4 / a8)
#   backward : dedup (a1) + segment-reduce (a6) + optimizer (a11-a13)
# --------------------------------------------------------------------------


def pooled_step(
    table,
    state,
    ids,
    offsets,
    row_base,
    batch_size,
    dim,
    pooled_grad,
    *,
    storage="bfloat16",
    pooling=POOLING_SUM,
    weights=None,
    optimizer="rowwise_adagrad",
    lr=0.01,
    eps=1e-8,
    beta1=0.9,
    beta2=0.999,
    normalization_steps=1,
    unit=REDUCE_UNIT,
):
    """Return ``(pooled, new_table, new_state, unique, inverse, first_indices)``.

    ``state`` is a dict: ``{"acc": [R]}`` for row-wise Adagrad,
    ``{"m": [R,D], "v": [R,D], "step": [R]}`` for Adam, ``{}`` for SGD.
    Keys are global rows ``row_base[t] + ids[i]``; dedup is first-occurrence
    over the concatenated (table-major) occurrence stream.
    """
    pooled = gather_pooled_csr(
        table, ids, offsets, row_base, batch_size, dim,
        storage=storage, pooling=pooling, weights=weights,
    )
    num_tables = int(np.asarray(row_base).size) - 1
    offsets = np.asarray(offsets, dtype=np.int64)
    lengths = np.diff(offsets)
    bag_of = np.repeat(np.arange(num_tables * batch_size), lengths)
    keys = row_base[bag_of // batch_size] + np.asarray(ids, dtype=np.int64)
    unique, inverse, first = unique_first_occurrence_sorted(keys)
    # per-occurrence gradient contribution (backward of the pooling)
    g = np.asarray(pooled_grad, dtype=np.float32).reshape(batch_size, num_tables, dim)
    g_bag = g.transpose(1, 0, 2).reshape(-1, dim)  # bag k = t*B + b
    contrib = g_bag[bag_of]
    if pooling == POOLING_WEIGHTED:
        contrib = (contrib * np.asarray(weights, np.float32)[:, None]).astype(np.float32)
    elif pooling == POOLING_MEAN:
        scale = np.maximum(lengths, 1).astype(np.float32)[bag_of]
        contrib = (contrib / scale[:, None]).astype(np.float32)
    perm, sk, starts = sorted_occurrences(keys)
    sums = segment_sums(contrib[perm], starts, perm.size, unit)
    rows = sk[starts]
    if normalization_steps != 1:
        sums = (sums / np.float32(normalization_steps)).astype(np.float32)
    new_table = np.array(table, copy=True)
    w = storage_to_f32(np.asarray(table)[rows], storage)
    new_state = {k: np.array(v, copy=True) for k, v in state.items()}
    if optimizer == "rowwise_adagrad":
        w2, acc2 = rowwise_adagrad_update(w, state["acc"][rows], sums, lr=lr, eps=eps)
        new_state["acc"][rows] = acc2
    elif optimizer == "adam":
        w2, m2, v2, s2 = adam_update(
            w, state["m"][rows], state["v"][rows], state["step"][rows], sums,
            lr=lr, beta1=beta1, beta2=beta2, eps=eps,
        )
        new_state["m"][rows], new_state["v"][rows], new_state["step"][rows] = m2, v2, s2
    elif optimizer == "sgd":
        w2 = sgd_update(w, sums, lr=lr)
    else:
        raise ValueError(optimizer)
    new_table[rows] = f32_to_storage(w2, storage)
    return pooled, new_table, new_state, unique, inverse, first


def pooled_grad_sums(ids, offsets, row_base, batch_size, dim, pooled_grad, *,
                     pooling=POOLING_SUM, weights=None, unit=REDUCE_UNIT):
    """Backward only (config 3): per-unique-key reduced gradient, first-occurrence order."""
    num_tables = int(np.asarray(row_base).size) - 1
    offsets = np.asarray(offsets, dtype=np.int64)
    lengths = np.diff(offsets)
    bag_of = np.repeat(np.arange(num_tables * batch_size), lengths)
    keys = row_base[bag_of // batch_size] + np.asarray(ids, dtype=np.int64)
    unique, inverse, first = unique_first_occurrence_sorted(keys)
    g = np.asarray(pooled_grad, dtype=np.float32).reshape(batch_size, num_tables, dim)
    contrib = g.transpose(1, 0, 2).reshape(-1, dim)[bag_of]
    if pooling == POOLING_WEIGHTED:
        contrib = (contrib * np.asarray(weights, np.float32)[:, None]).astype(np.float32)
    elif pooling == POOLING_MEAN:
        contrib = (contrib / np.maximum(lengths, 1).astype(np.float32)[bag_of][:, None]).astype(np.float32)
    perm, sk, starts = sorted_occurrences(keys)
    sums = segment_sums(contrib[perm], starts, perm.size, unit)
    # sorted-key order -> first-occurrence order
    order = np.argsort(sk[starts], kind="stable")
    by_key = dict(zip(sk[starts][order].tolist(), order.tolist()))
    out = sums[[by_key[int(k)] for k in unique.tolist()]] if unique.size else sums
    return unique, inverse, first, out


def ulp_distance_f32(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Distance in float32 units-in-the-last-place (monotone integer mapping)."""
    def key(x):
        i = np.ascontiguousarray(x, dtype=np.float32).view(np.int32).astype(np.int64)
        return np.where(i < 0, -(i & 0x7FFFFFFF), i)
    return np.abs(key(a) - key(b))


def storage_ulp_distance(a, b, storage: str) -> np.ndarray:
    """Distance in units of the storage dtype's last place."""
    if storage == "bfloat16":
        ia = np.asarray(a, np.uint16).astype(np.int64)
        ib = np.asarray(b, np.uint16).astype(np.int64)
    elif storage == "float16":
        ia = np.asarray(a, np.float16).view(np.uint16).astype(np.int64)
        ib = np.asarray(b, np.float16).view(np.uint16).astype(np.int64)
    else:
        return ulp_distance_f32(a, b)
    def key(i):
        return np.where(i & 0x8000, -(i & 0x7FFF), i)
    return np.abs(key(ia) - key(ib))


# --------------------------------------------------------------------------
# CSR-native ingest: dense positions of first occurrences
# (_unique_global_flat_positions, sparse_input.py:85-113; its helpers live in the
# absent fluxway.common.tensor_components, so this states the row-major offset of
# each flat value's nested path, pinned by the reference's vector
# tests/runtime/test_sparse_input_resources.py:77-105 and a dense brute force)
# --------------------------------------------------------------------------
def nested_global_positions(nested_splits, first_indices, widths, origin_indices) -> np.ndarray:
    """Flat index -> (row r0, j1..jL) -> origin[r0]*S0 + sum j_k*S_k (S: suffix products of
    widths); -1 where the path leaves the dense shape."""
    levels = len(nested_splits)
    strides = [1] * (levels + 1)
    for k in range(levels - 1, -1, -1):
        strides[k] = strides[k + 1] * int(widths[k])
    v = np.asarray(first_indices, dtype=np.int64).copy()
    pos = np.zeros(v.size, dtype=np.int64)
    ok = np.ones(v.size, dtype=bool)
    for k in range(levels - 1, -1, -1):
        sp = np.asarray(nested_splits[k], dtype=np.int64)
        inside = (v >= sp[0]) & (v < sp[-1]) & ok
        e = np.searchsorted(sp, v, side="right") - 1
        e = np.clip(e, 0, max(sp.size - 2, 0))
        j = v - sp[e]
        ok &= inside & (j < int(widths[k]))
        pos += np.where(ok, j * strides[k + 1], 0)
        v = np.where(ok, e, 0)
    origin = np.asarray(origin_indices, dtype=np.int64)
    ok &= v < origin.size
    pos += np.where(ok, origin[np.where(ok, v, 0)] * strides[0] if origin.size else 0, 0)
    return np.where(ok, pos, -1).astype(np.int32)


# --------------------------------------------------------------------------
# dynamic key -> row map (the dynamic store's lookup_or_insert)
# The reference drives an external store: lookup_or_insert(keys, dim)
# (dynamic_embedding.py:397-399) with new rows from Uniform(-0.01, 0.01)
# (:262-263).  This restates the HIP library's definition of it.
# --------------------------------------------------------------------------
_MIX1 = np.uint64(0xBF58476D1CE4E5B9)
_MIX2 = np.uint64(0x94D049BB133111EB)
_GOLDEN = np.uint64(0x9E3779B97F4A7C15)


def splitmix64_mix(z: np.ndarray) -> np.ndarray:
    """The SplitMix64 output function (Steele, Lea, Flood 2014) on uint64 arrays (wrapping)."""
    z = np.asarray(z, dtype=np.uint64)
    z = (z ^ (z >> np.uint64(30))) * _MIX1
    z = (z ^ (z >> np.uint64(27))) * _MIX2
    return z ^ (z >> np.uint64(31))


def keymap_initial_values(keys, dim: int, lo: float, hi: float, seed: int, storage: str) -> np.ndarray:
    """Initial row of each key: element c is ``lo + (hi - lo) * u`` (float32 operations) with
    ``u = (mix(mix(seed ^ key) + golden * (c + 1)) >> 40) * 2^-24``, then RNE to storage."""
    k = np.ascontiguousarray(keys, dtype=np.int64).view(np.uint64).reshape(-1, 1)
    cols = np.arange(1, dim + 1, dtype=np.uint64).reshape(1, -1)
    with np.errstate(over="ignore"):
        z = splitmix64_mix(splitmix64_mix(np.uint64(seed) ^ k) + _GOLDEN * cols)
    u = (z >> np.uint64(40)).astype(np.uint32).astype(np.float32) * np.float32(2.0 ** -24)
    flo, fhi = np.float32(lo), np.float32(hi)
    values = flo + (fhi - flo) * u
    return f32_to_storage(values.astype(np.float32), storage)


class KeyMap:
    """Key -> row map: new keys take rows count, count+1, ... in the order of their first
    occurrence in each call, until ``row_capacity`` rows are given out; keys left without a row
    are absent (row -1) and may get one in a later call."""

    def __init__(self, row_capacity: int):
        self.row_capacity = int(row_capacity)
        self.rows: dict[int, int] = {}

    def lookup_or_insert(self, keys, insert: bool = True):
        """Returns (rows int32 [-1 when absent], fresh bool: the key had no row before)."""
        keys = np.asarray(keys, dtype=np.int64).reshape(-1)
        rows = np.full(keys.size, -1, dtype=np.int32)
        fresh = np.zeros(keys.size, dtype=bool)
        before = dict(self.rows)
        for i, key in enumerate(keys.tolist()):
            if key == -(2 ** 63):
                continue  # not storable
            row = self.rows.get(key)
            if row is None and insert and len(self.rows) < self.row_capacity:
                row = len(self.rows)
                self.rows[key] = row
            if row is not None:
                rows[i] = row
                fresh[i] = key not in before
        return rows, fresh
