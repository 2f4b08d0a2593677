#!/usr/bin/env python3
"""Benchmark of the fused sparse-embedding step on one MI355X.

A step is one pass of the hot path over one batch: CSR pooled lookup
(forward), id dedup (sort / unique), and the deterministic segment-reduce
with the row-wise Adagrad update of the table rows (backward).  Default
workload: 26 tables (rows log-uniform in [1e3, 1e7]), dim 128, bf16 rows with
fp32 accumulation and fp32 Adagrad state, batch 65536, one id per table per
sample, Zipf(1.1) ids, synthetic fp32 N(0, 1e-3) pooled gradients.

Inputs are resident in HBM before timing.  Steps rotate over several
pre-generated id batches so the unique-row footprint exceeds the 256 MB
Infinity Cache.  HIP events on the shard's stream time each phase; the
reported step time is the median over the timed steps.  The forward phase is
exactly one kernel launch (the pooled gather), which the roofline entry
reports: algorithmic bytes of the launch / its event-timed duration.

Prints one JSON line (see ``--help``).  ``--gpus`` above 1 is rejected: this
build measures one GPU.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

METRIC = "pooled embedding rows/sec (fwd+bwd+update); achieved HBM GB/s vs 8 TB/s peak"
PEAK_HBM_GBS = 8000.0
STATE_BYTES = {"rowwise_adagrad": 4, "sgd": 0}
WORKLOAD_NAMES = {
    1: "1 table x 1e6 x 64 fp32, batch 4096, bags U[1,20], Zipf 1.05, row-wise Adagrad",
    2: "26 tables (rows log-uniform 1e3..1e7) x 128 bf16, batch 65536, bag 1, Zipf 1.1, row-wise Adagrad fp32 state",
    3: "8 tables x 5e6 x 64 fp16, batch 16384, bags geometric(30)<=500, Zipf 1.05, weighted-sum pooling, backward to reduced grads",
    4: "26 tables x 2e6 x 128 bf16, batch 65536, bags U[1,8], Zipf 1.3, row-wise Adagrad",
    5: "1 table x 1e8 x 128 bf16, Adam fp32 m/v, batch 131072, bags U[1,64], Zipf 1.05",
}


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def step_bytes(n: int, u: int, batch: int, tables: int, dim: int, s: int, weighted: bool,
               optimizer: str, g: int = 4) -> tuple[int, int, int]:
    """Algorithmic HBM bytes (forward, backward, update kernel) of one step.

    forward : ids N*8 + offsets T*(B+1)*4 + weights N*4 + unique rows U*D*s + pooled B*T*D*s
    backward: ids N*8 + offsets + weights + pooled grads B*T*D*g + unique U*8 + inverse N*4
              + rows 2*U*D*s + state 2*U*S   (S = 4 row-wise Adagrad, 2*D*4+4 Adam)
              (gradient-only: U*D*4 reduced gradients instead of rows and state)
    update kernel: grads B*T*D*g + rows 2*U*D*s + state 2*U*S + inverse N*4
    (g: bytes of a pooled gradient element, 4 for float32, 2 for the bfloat16 transport dtype)
    """
    offsets = tables * (batch + 1) * 4
    w = n * 4 if weighted else 0
    fwd = n * 8 + offsets + w + u * dim * s + batch * tables * dim * s
    if optimizer == "none":
        rows_state = u * dim * 4
    else:
        state = 2 * dim * 4 + 4 if optimizer == "adam" else STATE_BYTES[optimizer]
        rows_state = 2 * u * dim * s + 2 * u * state
    bwd = n * 8 + offsets + w + batch * tables * dim * g + u * 8 + n * 4 + rows_state
    update = batch * tables * dim * g + rows_state + n * 4
    return fwd, bwd, update


def update_kernel_bytes(w, s: int, g: int = 4) -> tuple[int, int]:
    """Algorithmic HBM bytes of the two update kernels for one batch ``w``.

    Keys are stably sorted; a key's positions inside one 64-position unit form one piece.
    A bag's gradient row is read once per kernel however many of that kernel's occurrences
    it holds (R_x: distinct bags among the occurrences of kind x).

    Optimizer updates (piece_sums_kernel, key_apply_kernel):
    piece_sums: R_multi * D*g gradient rows of keys with several occurrences + N * 4 sorted
                gradient rows + P_multi * D*4 piece rows written + N * 4 inverse
    key_apply : U * (2*D*s row read and write + 2*S state) + R_single * D*g
                + P_multi * D*4 piece rows read
    Reduced gradients (sums_kernel, apply_kernel; "long" keys cross a unit boundary or have
    more than 4 positions, the others are summed inside apply_kernel):
    sums : R_long * D*g + N_long * 4 row indices + P_long * D*4 partials
    apply: U * D*4 reduced rows written + R_short * D*g + N_short * 4 + U_long * D*4
    (g: bytes of a pooled gradient element)
    """
    import numpy as np

    keys = w.global_keys()
    dim = w.dim
    uniq, inverse, counts = np.unique(keys, return_inverse=True, return_counts=True)
    n = int(counts.sum())
    starts = np.cumsum(counts) - counts
    h = starts // 64
    last = (starts + counts - 1) // 64
    pieces = last - h + 1
    u = int(counts.size)
    bag = np.repeat(np.arange(w.num_tables * w.batch, dtype=np.int64), np.diff(w.offsets))
    inverse = inverse.reshape(-1)

    def bags_of(key_mask):
        return int(np.unique(bag[key_mask[inverse]]).size)

    if w.optimizer == "none":
        long_ = (h != last) | (counts > 4)
        n_long = int(counts[long_].sum())
        sums = bags_of(long_) * dim * g + n_long * 4 + int(pieces[long_].sum()) * dim * 4
        apply = u * dim * 4 + bags_of(~long_) * dim * g + (n - n_long) * 4 + int(long_.sum()) * dim * 4
        return sums, apply
    state = 2 * dim * 4 + 4 if w.optimizer == "adam" else STATE_BYTES[w.optimizer]
    multi = counts > 1
    p_multi = int(pieces[multi].sum())
    sums = bags_of(multi) * dim * g + n * 4 + p_multi * dim * 4 + n * 4
    apply = u * (2 * dim * s + 2 * state) + bags_of(~multi) * dim * g + p_multi * dim * 4
    return sums, apply


def kernel_traffic(config: int, kernel: str):
    """HBM bytes per launch of ``kernel`` on workload ``config`` from the committed counter runs.

    profiles/step_kernel_traffic.json holds, per workload, FETCH_SIZE and WRITE_SIZE (KiB per
    dispatch) of the step's kernels and the factors that map each counter onto the bytes of a
    plain device copy of known size.  None when the workload or kernel was not profiled.
    """
    path = ROOT / "profiles" / "step_kernel_traffic.json"
    if not path.exists():
        return None
    rec = json.loads(path.read_text()).get("workloads", {}).get(str(config))
    if rec is None or kernel not in rec.get("kernels", {}):
        return None
    k = rec["kernels"][kernel]
    return (k["fetch_kib"] * rec["fetch_scale"] + k["write_kib"] * rec["write_scale"]) * 1024.0


def _cpu_inputs(w):
    """Table, optimizer state and pooled gradient of one workload for the CPU restatement."""
    import numpy as np

    from oracle import cpu_step as C

    table = C.init_table(w.total_rows, w.dim, w.value_dtype, -w.init_range, w.init_range, 11)
    rng = np.random.default_rng(5)
    grad = (rng.standard_normal((w.batch, w.num_tables, w.dim), dtype=np.float32) * np.float32(1e-3))
    if w.optimizer == "adam":
        state = {"m": np.zeros((w.total_rows, w.dim), np.float32), "v": np.zeros((w.total_rows, w.dim), np.float32),
                 "step": np.zeros(w.total_rows, np.int32)}
    elif w.optimizer == "rowwise_adagrad":
        state = {"acc": np.zeros(w.total_rows, np.float32)}
    else:
        state = {}
    return table, state, grad


def _cpu_steps(w, inputs, seconds: float, max_steps: int, min_steps: int = 3) -> tuple[float, int]:
    """Median seconds per step of the oracle's C restatement of the reference CPU path."""
    from oracle import cpu_step as C

    table, state, grad = inputs
    times = []
    start = C.now()
    while (C.now() - start < seconds and len(times) < max_steps) or len(times) < min_steps:
        t0 = C.now()
        C.pooled_forward(table, w.value_dtype, w.dim, w.ids, w.offsets, w.num_tables, w.batch, w.row_base(),
                         w.pooling, w.weights)
        C.pooled_backward(table, w.value_dtype, w.dim, state, w.optimizer, w.ids, w.offsets, w.num_tables,
                          w.batch, w.row_base(), grad, w.pooling, w.weights)
        times.append(C.now() - t0)
    return statistics.median(times), len(times)


def cpu_baseline(config: int, seconds: float) -> dict:
    """Time the oracle's C restatement of the reference CPU path on host cores: the benched
    workload with every host thread and with one, and workload 1 (the reference's own
    CPU-sized case) with every thread."""
    from flare_amd.workload import make_workload
    from oracle import cpu_step as C

    cores = C.threads()
    w = make_workload(config, batch_index=0)
    inputs = _cpu_inputs(w)
    med, steps = _cpu_steps(w, inputs, seconds, 50)
    C.set_threads(1)
    try:
        med1, steps1 = _cpu_steps(w, inputs, seconds / 4, 3, min_steps=1)
    finally:
        C.set_threads(cores)
    del inputs
    w1 = make_workload(1, batch_index=0)
    med_w1, steps_w1 = _cpu_steps(w1, _cpu_inputs(w1), seconds / 8, 200)
    return {
        "value": w.batch * w.num_tables / med,
        "unit": "pooled rows/s",
        "cores": cores,
        "kind": "port",
        "sample": f"C/OpenMP restatement of the reference Numba path (pooled gather, serial per-table "
                  f"first-occurrence hash dedup, keyed scatter, optimizer); workload {config} full batch "
                  f"of {w.batch} x {w.num_tables} bags, median of {steps} steps",
        "ms_per_step": med * 1e3,
        "one_thread": {"value": w.batch * w.num_tables / med1, "ms_per_step": med1 * 1e3, "steps": steps1},
        "workload_1": {"value": w1.batch * w1.num_tables / med_w1, "ms_per_step": med_w1 * 1e3,
                       "steps": steps_w1, "cores": cores,
                       "workload": "1 table of 1e6 rows x 64 fp32, batch 4096, bags U[1,20], Zipf 1.05, "
                                   "row-wise Adagrad"},
    }


def full_size_check(shard, plan, w, grad, grad_out, none_opt, sample: int = 4096, seed: int = 7) -> dict:
    """One more full-size step of ``plan``, checked (the oracle is the checker here, after timing).

    - dedup invariants over all N occurrences: ``unique[inverse] == keys``,
      ``keys[first] == unique``, ``first`` strictly increasing, ``U`` = distinct keys;
    - ``sample`` random bags: pooled rows bit-exact against the oracle's pooling of the
      rows they read (taken from the table before the step);
    - ``sample`` random unique keys: their updated rows (within 1 ulp of the storage dtype)
      and optimizer state (rtol 1e-5), or their reduced gradients (bit-exact), against the
      oracle's segment sums in the same unit order and its optimizer;
    - ``sample`` random rows no id touched: unchanged.
    Rows are compared as gathered before and after the step, so no table is copied whole.
    """
    import numpy as np
    import torch

    from flare_amd import _native
    from oracle import sparse_oracle as O

    dev = shard.device
    stream = shard.stream
    rng = np.random.default_rng(seed)
    keys = w.global_keys()
    lengths = np.diff(w.offsets)
    bag_of = np.repeat(np.arange(w.num_tables * w.batch, dtype=np.int64), lengths)
    perm, sk, starts = O.sorted_occurrences(keys)
    ends = np.append(starts[1:], perm.size)
    seg_keys = sk[starts]
    pick = np.sort(rng.choice(starts.size, size=min(sample, starts.size), replace=False))
    check_rows = seg_keys[pick]
    touched = np.zeros(w.total_rows, dtype=bool)
    touched[seg_keys] = True
    free = np.nonzero(~touched)[0]
    still_rows = rng.choice(free, size=min(sample, free.size), replace=False) if free.size else free
    nbags = w.num_tables * w.batch
    bags = np.sort(rng.choice(nbags, size=min(sample, nbags), replace=False))
    st = shard.state

    def rows_of(t, rows):
        if t is None:
            return None
        idx = torch.from_numpy(np.asarray(rows, np.int64)).to(dev)
        return t.index_select(0, idx)

    def host(t):
        if t is None:
            return None
        if t.dtype == torch.bfloat16:
            return t.view(torch.int16).cpu().numpy().view(np.uint16)
        return t.cpu().numpy()

    pooled_row = bags if shard.layout == "table_major" else (bags % w.batch) * w.num_tables + bags // w.batch
    with torch.cuda.stream(stream):
        bag_rows = np.unique(keys[np.concatenate([np.arange(w.offsets[k], w.offsets[k + 1]) for k in bags])])
        before = {name: host(rows_of(t, check_rows)) for name, t in
                  (("table", st.table), ("s0", st.state0), ("s1", st.state1), ("step", st.step))}
        pool_src = host(rows_of(st.table, bag_rows))
        still_before = host(rows_of(st.table, still_rows))
        plan.forward()
        plan.dedup()
        plan.apply(grad, grad_out=grad_out, optimizer=none_opt)
        after = {name: host(rows_of(t, check_rows)) for name, t in
                 (("table", st.table), ("s0", st.state0), ("s1", st.state1), ("step", st.step))}
        still_after = host(rows_of(st.table, still_rows))
        pooled = host(plan.pooled.reshape(-1, w.dim)[torch.from_numpy(pooled_row).to(dev)])
    errors = int(_native.library().flare_take_device_errors(int(stream.cuda_stream)))
    u = int(plan.unique_count.item())
    unique = plan.unique[:u].cpu().numpy()
    inverse = plan.inverse[:w.num_ids].cpu().numpy()
    first = plan.first_indices[:u].cpu().numpy()
    out = {"device_errors": errors, "occurrences": int(keys.size), "unique": u}
    out["unique_count_ok"] = u == int(starts.size)
    out["unique_inverse_ok"] = bool(np.array_equal(unique[inverse], keys))
    out["first_indices_ok"] = bool(np.array_equal(keys[first], unique) and np.all(np.diff(first) > 0))
    # pooled rows of the sampled bags: the oracle pools the same rows (compact table)
    sub_off = np.zeros(bags.size + 1, np.int64)
    sub_off[1:] = np.cumsum(lengths[bags])
    sub_keys = np.concatenate([keys[w.offsets[k]:w.offsets[k + 1]] for k in bags])
    sub_ids = np.searchsorted(bag_rows, sub_keys)
    sub_w = None if w.weights is None else np.concatenate([w.weights[w.offsets[k]:w.offsets[k + 1]] for k in bags])
    expected = O.gather_pooled_csr(pool_src, sub_ids, sub_off, np.asarray([0, bag_rows.size], np.int64), bags.size,
                                   w.dim, storage=w.value_dtype, pooling=w.pooling, weights=sub_w)
    out["sampled_bags"] = int(bags.size)
    out["pooled_bit_exact"] = bool(np.array_equal(pooled, expected.reshape(bags.size, w.dim)))
    # reduced gradients of the sampled keys, in the kernels' unit order
    positions = np.unique(np.concatenate([np.arange(a, e) for a, e in zip(starts[pick], ends[pick])]))
    occ = perm[positions]
    grow = bag_of[occ] if shard.layout == "table_major" else \
        (bag_of[occ] % w.batch) * w.num_tables + bag_of[occ] // w.batch
    g_rows = grad.reshape(-1, w.dim).index_select(0, torch.from_numpy(grow).to(dev)).float().cpu().numpy()
    if w.pooling == "weighted":
        g_rows = (g_rows * w.weights[occ][:, None]).astype(np.float32)
    elif w.pooling == "mean":
        g_rows = (g_rows / np.maximum(lengths[bag_of[occ]], 1).astype(np.float32)[:, None]).astype(np.float32)
    sums = O.segment_sums_selected(lambda pos: g_rows[np.searchsorted(positions, pos)], starts[pick], ends[pick],
                                   w.dim)
    out["sampled_keys"] = int(pick.size)
    if none_opt is not None:  # reduced gradients in first-occurrence order
        rank = np.searchsorted(np.sort(unique), check_rows)
        order = np.argsort(unique, kind="stable")
        got = grad_out[:u][torch.from_numpy(order[rank]).to(dev)].cpu().numpy()
        out["reduced_grad_bit_exact"] = bool(np.array_equal(got, sums))
        ok_rows = out["reduced_grad_bit_exact"]
    else:
        w0 = O.storage_to_f32(before["table"], w.value_dtype)
        if w.optimizer == "adam":
            w1, m1, v1, s1 = O.adam_update(w0, before["s0"], before["s1"], before["step"], sums, lr=0.01)
            state_pairs = [(after["s0"], m1), (after["s1"], v1)]
            steps_ok = bool(np.array_equal(after["step"], s1))
        else:
            w1, acc1 = O.rowwise_adagrad_update(w0, before["s0"], sums, lr=0.01, eps=1e-8)
            state_pairs = [(after["s0"], acc1)]
            steps_ok = True
        ulps = O.storage_ulp_distance(after["table"], O.f32_to_storage(w1, w.value_dtype), w.value_dtype)
        rel = max(float(np.max(np.abs(a - b) / np.maximum(np.abs(b), 1e-30))) for a, b in state_pairs)
        out["rows_max_ulp"] = int(ulps.max())
        out["state_max_rel_err"] = rel
        ok_rows = out["rows_max_ulp"] <= 1 and rel <= 1e-5 and steps_ok
    out["untouched_rows"] = int(still_rows.size)
    out["untouched_rows_unchanged"] = bool(np.array_equal(still_before, still_after))
    out["passed"] = bool(errors == 0 and out["unique_count_ok"] and out["unique_inverse_ok"] and
                         out["first_indices_ok"] and out["pooled_bit_exact"] and ok_rows and
                         out["untouched_rows_unchanged"])
    return out


def _int64_key_sets(batches: int) -> list:
    """Unique ids of workload 5 batches (1e8-id space, 131072 bags of U[1,64] Zipf(1.05) ids)
    in first-occurrence order, mixed by the SplitMix64 output function into arbitrary int64
    keys (numpy arrays)."""
    import numpy as np

    from flare_amd.workload import make_workload

    out = []
    for k in range(batches):
        ids = make_workload(5, batch_index=k).ids
        _, first = np.unique(ids, return_index=True)
        uids = ids[np.sort(first)].astype(np.uint64)
        with np.errstate(over="ignore"):
            z = (uids ^ (uids >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
            z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
            z = z ^ (z >> np.uint64(31))
        keys = z.view(np.int64)
        out.append(keys[keys != np.iinfo(np.int64).min].copy())
    return out


def _event_ms(stream, fn, steps: int, warmup: int) -> float:
    """Median over ``steps`` calls of ``fn`` of the time between events recorded on ``stream``
    around each call (after ``warmup`` untimed calls)."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for a, b in events:
        a.record(stream)
        fn()
        b.record(stream)
    torch.cuda.synchronize()
    return statistics.median(a.elapsed_time(b) for a, b in events)


def ingest_main(args) -> int:
    """CSR-native ingest: dense global positions of each unique id's first occurrence.

    One ragged feature of workload 5 (131072 rows of U[1,64] ids, dense width 64): the first
    occurrences of its unique ids (about 1.1M of 4.3M) are mapped through the row splits and
    the rows' origins (``origin_indices``: this worker's rows at offset 131072 of the global
    batch) to ``origin*64 + j``.  A second line runs a two-level nesting (rows of up to 8
    lists of up to 8 ids) of the same ids.
    """
    import numpy as np
    import torch

    from flare_amd import _native
    from flare_amd.workload import make_workload

    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    w = make_workload(5)
    ids = w.ids
    _, first = np.unique(ids, return_index=True)
    first = np.sort(first).astype(np.int64)
    rows = w.batch
    origin = (np.arange(rows, dtype=np.int64) + rows)
    # two levels: each bag of <= 64 ids split into lists of <= 8
    lengths = np.diff(w.offsets)
    inner = []
    outer = np.zeros(rows + 1, np.int64)
    for b, ln in enumerate(lengths.tolist()):
        parts = [8] * (ln // 8) + ([ln % 8] if ln % 8 else [])
        inner.extend(parts)
        outer[b + 1] = outer[b] + len(parts)
    inner_splits = np.zeros(len(inner) + 1, np.int64)
    inner_splits[1:] = np.cumsum(inner)
    cases = [("1 level, width 64", [np.asarray(w.offsets, np.int64)], [64]),
             ("2 levels, widths 8 x 8", [outer, inner_splits], [8, 8])]
    stream = torch.cuda.Stream(device)
    for name, splits, widths in cases:
        d_splits = [torch.from_numpy(sp).to(device) for sp in splits]
        d_first = torch.from_numpy(first).to(device)
        d_origin = torch.from_numpy(origin).to(device)
        out = torch.empty(first.size, dtype=torch.int32, device=device)
        levels = len(splits)
        ptrs = (ctypes.c_void_p * levels)(*[t.data_ptr() for t in d_splits])
        lens = (ctypes.c_int64 * levels)(*[int(t.numel()) for t in d_splits])
        dims = (ctypes.c_int64 * levels)(*widths)

        def call():
            _native.call("flare_nested_global_positions", d_first.data_ptr(), int(first.size), levels,
                         ctypes.cast(ptrs, ctypes.c_void_p), ctypes.cast(lens, ctypes.c_void_p),
                         d_origin.data_ptr(), int(origin.size), ctypes.cast(dims, ctypes.c_void_p),
                         out.data_ptr(), int(stream.cuda_stream))

        ms = _event_ms(stream, call, args.steps, args.warmup)
        got = out.cpu().numpy()
        # algorithmic bytes: each first index read (8) and position written (4), one origin
        # read (8) and, per level, the two split entries that bound its list (16)
        per_index = 8 + 4 + 8 + 16 * levels
        gbs = first.size * per_index / (ms * 1e-3) / 1e9
        line = {
            "metric": "nested global positions per second (CSR-native ingest)",
            "value": first.size / (ms * 1e-3),
            "unit": "positions/s",
            "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_call": ms,
            "higher_is_better": True, "dtype": "int64",
            "data": "synthetic (workload 5 ids)",
            "config": {"workload": f"{first.size} first occurrences of {ids.size} ids in {rows} rows, {name}"},
            "roofline": {"kernel": "positions_kernel", "bound": "hbm", "achieved": gbs, "peak": 8000.0,
                         "unit": "GB/s", "frac": gbs / 8000.0, "traffic": None,
                         "algorithmic_bytes_per_position": per_index},
        }
        if not args.no_cpu_baseline:
            from oracle import sparse_oracle as O  # the CPU leg only

            t0 = time.perf_counter()
            reps = 0
            while True:
                exp = O.nested_global_positions(splits, first, widths, origin)
                reps += 1
                if time.perf_counter() - t0 > 3.0 or reps >= 20:
                    break
            cpu_s = (time.perf_counter() - t0) / reps
            if not np.array_equal(exp, got):
                raise SystemExit(f"ingest positions differ from the oracle ({name})")
            line["cpu_baseline"] = {"value": first.size / cpu_s, "unit": "positions/s", "cores": 1,
                                    "kind": "port", "sample": f"the same input, numpy, {reps} calls"}
        print(json.dumps(line), flush=True)
    return 0


def pages_main(args) -> int:
    """Checkpoint page images of a dynamic store: export and import of every stored row.

    A 128-wide bf16 table under Adam holds the int64 keys of four workload 5 batches (about
    4M keys).  The device part of an export is the key map export plus the gathers of values,
    ``m``, ``v`` and step counters into page buffers; of an import, the key lookup plus the
    scatters back.  Both are timed with events; the whole ``export_page_images`` /
    ``import_page_images`` calls (pages of 1M keys, host numpy arrays: PCIe-inclusive) are
    timed by the wall clock beside them.
    """
    import numpy as np
    import torch

    from flare_amd.conversion import contiguous
    from flare_amd.store import Adam, DynamicEmbeddingStore

    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    dim = 128
    keys = np.unique(np.concatenate(_int64_key_sets(4)))
    store = DynamicEmbeddingStore(int(keys.size) + 1024, [dim], value_dtype="bfloat16", optimizer=Adam(), seed=5)
    d_keys = torch.from_numpy(keys).to(device)
    for lo in range(0, keys.size, 1 << 20):
        store.lookup_or_insert(d_keys[lo:lo + (1 << 20)], dim)
    store.synchronize()
    table = store.tables[dim]
    n = store.size(dim)
    stream = store.stream
    values = torch.empty((n, dim), dtype=table.table.dtype, device=device)
    m = torch.empty((n, dim), dtype=torch.float32, device=device)
    v = torch.empty((n, dim), dtype=torch.float32, device=device)
    steps = torch.empty(n, dtype=torch.int32, device=device)
    stored = {}

    def export_device():
        with torch.cuda.stream(stream):
            k, rows = store._stored(dim)
            stored["keys"], stored["rows"] = k, contiguous(rows)
            store._copy_rows(table.table, values, stored["rows"], None, n)
            store._copy_rows(table.state0, m, stored["rows"], None, n)
            store._copy_rows(table.state1, v, stored["rows"], None, n)
            store._copy_rows(table.step, steps, stored["rows"], None, n)

    def import_device():
        with torch.cuda.stream(stream):
            rows = store._rows_of(stored["keys"], dim, insert=True)
            store._copy_rows(values, table.table, None, rows, n)
            store._copy_rows(m, table.state0, None, rows, n)
            store._copy_rows(v, table.state1, None, rows, n)
            store._copy_rows(steps, table.step, None, rows, n)

    export_ms = _event_ms(stream, export_device, args.steps, args.warmup)
    import_ms = _event_ms(stream, import_device, args.steps, args.warmup)
    t0 = time.perf_counter()
    pages = store.export_page_images()
    export_wall = time.perf_counter() - t0
    t0 = time.perf_counter()
    store.import_page_images(pages)
    import_wall = time.perf_counter() - t0
    slots = store.maps[dim].slots
    # per key: value row 2*256 B (read + write), m and v 2*512 B each, step 2*4 B; the export
    # also writes key (8) and row (4) and reads every map slot (16 B) once, the import reads
    # the key (8), probes its slot (16) and writes the row (4)
    row_bytes = 2 * (dim * 2 + 2 * dim * 4 + 4)
    export_bytes = n * (row_bytes + 12) + 16 * slots
    import_bytes = n * (row_bytes + 28)
    for name, ms, nbytes, wall in (("export", export_ms, export_bytes, export_wall),
                                   ("import", import_ms, import_bytes, import_wall)):
        gbs = nbytes / (ms * 1e-3) / 1e9
        print(json.dumps({
            "metric": f"checkpoint page image {name} rows/s (device part)",
            "value": n / (ms * 1e-3), "unit": "rows/s",
            "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_call": ms,
            "higher_is_better": True, "dtype": "bf16 rows, fp32 Adam state",
            "data": "synthetic (workload 5 unique ids of 4 batches as int64 keys)",
            "config": {"workload": f"{n} keys, 128-wide bf16 table, Adam, map of {slots} slots"},
            "host_inclusive_s": wall, "host_inclusive_rows_per_s": n / wall,
            "roofline": {"kernel": "whole device part", "bound": "hbm", "achieved": gbs, "peak": 8000.0,
                         "unit": "GB/s", "frac": gbs / 8000.0, "traffic": None,
                         "algorithmic_bytes": nbytes},
        }), flush=True)
    return 0


def row_gather_main(args) -> int:
    """Random-row gather rate of this GPU, the ceiling of the update's gradient gather.

    ``flare_copy_rows`` gathers the 1.26M rows that sums_kernel reads per step on the default
    workload (long keys' occurrences) at random from a buffer the size of the fp32 pooled
    gradient (65536 x 26 rows of 512 bytes, 872 MB) into a dense buffer.  Also 256-byte rows
    (bf16 table rows) from a 5.9 GB buffer, as the apply kernel reads them.
    """
    import torch

    from flare_amd import _native

    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    stream = torch.cuda.Stream(device)
    gen = torch.Generator(device=device)
    gen.manual_seed(4)
    cases = [("512-byte rows of an 872 MB buffer (fp32 gradient rows)", 65536 * 26, 512, 1_260_000),
             ("256-byte rows of a 5.9 GB buffer (bf16 table rows)", 23_100_000, 256, 322_463)]
    for name, rows, row_bytes, n in cases:
        with torch.cuda.stream(stream):
            src = torch.empty(rows * row_bytes // 4, dtype=torch.float32, device=device).uniform_(generator=gen)
            dst = torch.empty(n * row_bytes // 4, dtype=torch.float32, device=device)
            index = torch.randint(0, rows, (n,), generator=gen, device=device, dtype=torch.int32)

        def call():
            _native.call("flare_copy_rows", src.data_ptr(), rows, dst.data_ptr(), n, row_bytes,
                         index.data_ptr(), None, n, int(stream.cuda_stream))

        ms = _event_ms(stream, call, args.steps, args.warmup)
        moved = n * (2 * row_bytes + 4)  # row read at random, written densely, index read
        print(json.dumps({
            "metric": "random row gather GB/s (flare_copy_rows)", "value": moved / (ms * 1e-3) / 1e9,
            "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_call": ms,
            "higher_is_better": True, "dtype": "raw bytes", "data": "synthetic (uniform random row indices)",
            "config": {"workload": f"{n} {name}"},
            "read_gbs": n * row_bytes / (ms * 1e-3) / 1e9, "rows_per_s": n / (ms * 1e-3),
        }), flush=True)
        del src, dst, index
        torch.cuda.empty_cache()
    return 0


def ceiling_main(args) -> int:
    """What plain streaming kernels reach on this GPU over 1 GiB: the ceiling the step's
    kernels are measured against.

    write: ``flare_zero_bytes`` (16-byte stores); copy: ``flare_copy_rows`` of one contiguous
    block (16-byte loads and stores, reported as bytes read + written); read:
    ``flare_check_finite`` over 1 GiB of float32 (16-byte loads, one flag written); and
    PyTorch's own ``copy_`` and ``sum`` beside them.  Each is the median of ``--steps`` calls
    timed with events.
    """
    import torch

    from flare_amd import _native

    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    stream = torch.cuda.Stream(device)
    nbytes = 1 << 30
    with torch.cuda.stream(stream):
        src = torch.empty(nbytes // 4, dtype=torch.float32, device=device).uniform_()
        dst = torch.empty_like(src)
        flag = torch.empty(1, dtype=torch.int32, device=device)
    s = int(stream.cuda_stream)
    cases = [
        ("write", nbytes, lambda: _native.call("flare_zero_bytes", dst.data_ptr(), nbytes, s)),
        ("copy", 2 * nbytes, lambda: _native.call("flare_copy_rows", src.data_ptr(), nbytes // 4096, dst.data_ptr(),
                                                  nbytes // 4096, 4096, None, None, nbytes // 4096, s)),
        ("read", nbytes, lambda: _native.call("flare_check_finite", src.data_ptr(), _native.FLOAT32, nbytes // 4,
                                              flag.data_ptr(), s)),
        ("torch copy_", 2 * nbytes, lambda: dst.copy_(src)),
        ("torch sum", nbytes, lambda: src.sum()),
    ]
    for name, moved, fn in cases:
        with torch.cuda.stream(stream):
            ms = _event_ms(stream, fn, args.steps, args.warmup)
        gbs = moved / (ms * 1e-3) / 1e9
        print(json.dumps({
            "metric": f"1 GiB {name} GB/s", "value": gbs, "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_call": ms, "higher_is_better": True, "dtype": "raw bytes",
            "data": "synthetic (uniform fp32)", "config": {"workload": f"{name} of 1 GiB"},
            "fraction_of_peak": gbs / PEAK_HBM_GBS,
        }), flush=True)
    return 0


def keymap_main(args) -> int:
    """Dynamic store: lookup_or_insert of one step's unique keys into a 128-wide bf16 table.

    Keys are the unique ids of workload 5 batches (1e8-id space, 131072 bags of U[1,64]
    Zipf(1.05) ids), in first-occurrence order, mixed into arbitrary int64 keys.  The first
    call inserts every key; the timed calls rotate over the batches once all are inserted.
    """
    import torch

    from flare_amd.store import DynamicEmbeddingStore, Sgd

    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    dim, batches = 128, max(2, min(args.batches, 4))
    key_sets = [torch.from_numpy(k).to(device) for k in _int64_key_sets(batches)]
    total = len(torch.unique(torch.cat(key_sets)))
    # load every kernel of the path once (a separate small store), so the timed first insert
    # does not include code-object loading
    warm = DynamicEmbeddingStore(4096, [dim], value_dtype="bfloat16", optimizer=Sgd(), seed=4)
    warm.lookup_or_insert(key_sets[0][:1000], dim)
    warm.lookup_or_insert(key_sets[0][:1000], dim)
    warm.synchronize()
    del warm
    store = DynamicEmbeddingStore(total + 1024, [dim], value_dtype="bfloat16", optimizer=Sgd(), seed=3)
    stream = store.stream
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    torch.cuda.synchronize()
    ev[0].record(stream)
    store.lookup_or_insert(key_sets[0], dim)
    ev[1].record(stream)
    torch.cuda.synchronize()
    insert_ms = ev[0].elapsed_time(ev[1])
    for ks in key_sets[1:]:
        store.lookup_or_insert(ks, dim)
    for i in range(args.warmup):
        store.lookup_or_insert(key_sets[i % batches], dim)
    torch.cuda.synchronize()
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    nkeys = []
    for i in range(args.steps):
        ks = key_sets[i % batches]
        nkeys.append(ks.numel())
        events[i][0].record(stream)
        store.lookup_or_insert(ks, dim)
        events[i][1].record(stream)
    torch.cuda.synchronize()
    ms = [a.elapsed_time(b) for a, b in events]
    med = statistics.median(ms)
    keys_per_call = statistics.median(nkeys)
    per_key = 8 + 12 + 4 + 2 * dim * 2  # key in, map slot (key + row word), row out, row read + values out
    gbs = keys_per_call * per_key / (med * 1e-3) / 1e9
    print(json.dumps({
        "metric": "dynamic store lookup_or_insert keys/s (steady state, keys present)",
        "value": keys_per_call / (med * 1e-3),
        "unit": "keys/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_call": med,
        "higher_is_better": True,
        "dtype": "bf16 rows",
        "data": "synthetic (workload 5 unique ids per batch, splitmix64-mixed into int64 keys)",
        "config": {"workload": f"{keys_per_call:.0f} unique int64 keys per call, 128-wide bf16 table of "
                               f"{store.tables[dim].rows} rows, map of {store.maps[dim].slots} slots",
                   "batches": batches, "keys_stored": store.size(dim)},
        "first_insert_ms": insert_ms,
        "first_insert_keys": int(key_sets[0].numel()),
        "roofline": {"kernel": "whole call (probe + values kernels)", "bound": "hbm", "achieved": gbs,
                     "peak": 8000.0, "unit": "GB/s", "frac": gbs / 8000.0, "traffic": None,
                     "algorithmic_bytes_per_key": per_key},
    }), flush=True)
    return 0


def dynamic_main(args) -> int:
    """The pooled step over int64 keys (DynamicEmbeddingStore): workload 2's ids mixed into
    arbitrary int64 keys, one 128-wide bf16 table with row-wise Adagrad shared by the 26
    features.  A step is lookup_pooled (key map lookup_or_insert of every occurrence, then the
    pooled gather) and apply_pooled_gradients (key map lookup, dedup, segment sums, update)."""
    import numpy as np
    import torch

    from flare_amd import _native
    from flare_amd.store import DynamicEmbeddingStore, RowWiseAdagrad, Uniform
    from flare_amd.workload import make_workload

    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    batches = max(2, min(args.batches, 4))
    sets = []
    for k in range(batches):
        w = make_workload(2, batch_index=k)
        g = w.global_keys().astype(np.uint64)
        with np.errstate(over="ignore"):
            z = (g ^ (g >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
            z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
            z = z ^ (z >> np.uint64(31))
        keys = z.view(np.int64)
        keys = np.where(keys == np.iinfo(np.int64).min, 0, keys)
        sets.append((torch.from_numpy(keys).to(device), torch.from_numpy(w.offsets).to(device)))
    batch, features, dim = w.batch, w.num_tables, w.dim
    total = len(torch.unique(torch.cat([k for k, _ in sets])))
    store = DynamicEmbeddingStore(total + 4096, [dim], value_dtype="bfloat16",
                                  optimizer=RowWiseAdagrad(lr=0.01, eps=1e-8), initializer=Uniform(-0.01, 0.01),
                                  seed=5)
    grad = torch.empty((features, batch, dim), dtype=torch.float32, device=device).normal_(0, 1e-3)
    grad = grad.to(torch.bfloat16)
    stream = store.stream

    def step(i):
        keys, offsets = sets[i % batches]
        store.lookup_pooled(keys, offsets, batch, dim)
        store.apply_pooled_gradients(keys, offsets, batch, grad, dim)

    for i in range(max(args.warmup, batches)):
        step(i)
    torch.cuda.synchronize()
    lib = _native.library()
    lib.flare_take_device_errors(int(stream.cuda_stream))
    events = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(args.steps)]
    with torch.cuda.stream(stream):
        for i in range(args.steps):
            keys, offsets = sets[i % batches]
            events[i][0].record(stream)
            store.lookup_pooled(keys, offsets, batch, dim)
            events[i][1].record(stream)
            store.apply_pooled_gradients(keys, offsets, batch, grad, dim)
            events[i][2].record(stream)
    torch.cuda.synchronize()
    errors = int(lib.flare_take_device_errors(int(stream.cuda_stream)))
    fwd = statistics.median(e[0].elapsed_time(e[1]) for e in events)
    bwd = statistics.median(e[1].elapsed_time(e[2]) for e in events)
    ms = statistics.median(e[0].elapsed_time(e[2]) for e in events)
    rows = features * batch
    print(json.dumps({
        "metric": "pooled embedding rows/sec (fwd+bwd+update) over int64 keys (dynamic store)",
        "value": rows / (ms * 1e-3), "unit": "pooled rows/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True, "dtype": "f32 (bf16 rows, bf16 pooled grads)",
        "data": "synthetic (workload 2 ids mixed by splitmix64 into int64 keys, N(0,1e-3) pooled grads)",
        "config": {"workload": "26 features x batch 65536, one int64 key per bag, one 128-wide bf16 table "
                               f"of {store.tables[dim].rows} rows with row-wise Adagrad, key map of "
                               f"{store.maps[dim].slots} slots", "keys_stored": store.size(dim),
                   "rotated_batches": batches},
        "phases_ms": {"lookup_pooled": fwd, "apply_pooled_gradients": bwd},
        "device_errors": errors,
    }), flush=True)
    return 0 if errors == 0 else 1


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", type=int, default=2, choices=[1, 2, 3, 4, 5])
    ap.add_argument("--batches", type=int, default=8, help="pre-generated id batches to rotate over")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-check", action="store_true",
                    help="skip the full-size correctness check of one more step after timing")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="before timing, run a plain device-to-device copy of this many MiB three times "
                         "(a kernel of known traffic, to scale FETCH_SIZE / WRITE_SIZE counters)")
    ap.add_argument("--layout", choices=["table_major", "sample_major"], default="table_major",
                    help="pooled row layout: [T, B, D] (the T per-table outputs one after the other) or [B, T, D]")
    ap.add_argument("--grad-dtype", choices=["auto", "float32", "bfloat16"], default="auto",
                    help="dtype of the pooled gradient handed to the update. auto: bfloat16 for bf16/fp16 "
                         "tables (the gradient transport dtype of the reference's BF16 and FP16 precision "
                         "policies, src/flare/jax/training/precision.py:62-69, cast before the gradient "
                         "leaves the JAX worker, train_worker.py:467-474), float32 for float32 tables")
    ap.add_argument("--order", choices=["pipelined", "dedup-first", "forward-first"], default="pipelined",
                    help="pipelined: each step runs its forward, then its update on the shard's stream while "
                         "the next batch's dedup runs on a second stream (the reference computes unique ids in "
                         "its input worker, ahead of the step: src/flare/runtime/fluxway/workers/"
                         "sparse_input.py:333-349); a step ends when both are done, so every timed step holds "
                         "one forward, one dedup and one update.  dedup-first / forward-first: the three "
                         "phases one after another on one stream")
    ap.add_argument("--overlap", action="store_true",
                    help="run the dedup (ids only) on a second stream, concurrent with the forward")
    ap.add_argument("--keymap", action="store_true",
                    help="measure the dynamic store's key map (lookup_or_insert) instead of the pooled step")
    ap.add_argument("--dynamic", action="store_true",
                    help="measure the pooled step over int64 keys through the dynamic store instead")
    ap.add_argument("--ingest", action="store_true",
                    help="measure CSR-native ingest (nested global positions) instead of the pooled step")
    ap.add_argument("--row-gather", action="store_true",
                    help="measure this GPU's random-row gather rate (the update's gradient gather ceiling)")
    ap.add_argument("--ceiling", action="store_true",
                    help="measure this GPU's streaming ceilings (1 GiB write, copy, read) instead of the pooled step")
    ap.add_argument("--pages", action="store_true",
                    help="measure checkpoint page image export/import instead of the pooled step")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only (the tables of one worker's shard on one MI355X); "
              f"--gpus {args.gpus} is not supported (one process, one GPU)", file=sys.stderr)
        return 2

    if args.keymap:
        return keymap_main(args)
    if args.dynamic:
        return dynamic_main(args)
    if args.ingest:
        return ingest_main(args)
    if args.pages:
        return pages_main(args)
    if args.row_gather:
        return row_gather_main(args)
    if args.ceiling:
        return ceiling_main(args)

    import torch

    from flare_amd import _native
    from flare_amd.store import Adam, PooledStepPipeline, PooledTableShard, RowWiseAdagrad, Uniform
    from flare_amd.workload import make_workload

    assert torch.cuda.is_available(), "bench.py needs a ROCm GPU"
    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    config = args.config
    t_setup = time.time()
    batches = [make_workload(config, batch_index=k) for k in range(args.batches)]
    w0 = batches[0]
    s = {"float32": 4, "float16": 2, "bfloat16": 2}[w0.value_dtype]
    optimizer = {"rowwise_adagrad": RowWiseAdagrad(lr=0.01, eps=1e-8), "adam": Adam(lr=0.01),
                 "none": RowWiseAdagrad(lr=0.01, eps=1e-8)}[w0.optimizer]
    shard = PooledTableShard(w0.table_rows, w0.dim, value_dtype=w0.value_dtype, optimizer=optimizer,
                             initializer=Uniform(-w0.init_range, w0.init_range), seed=1, layout=args.layout)
    plans = [shard.plan_step(b.ids, b.offsets, b.batch, pooling=b.pooling, per_sample_weights=b.weights)
             for b in batches]
    gen = torch.Generator(device=device)
    gen.manual_seed(2)
    grad_dtype = args.grad_dtype
    if grad_dtype == "auto":
        grad_dtype = "float32" if w0.value_dtype == "float32" else "bfloat16"
    g_bytes = 4 if grad_dtype == "float32" else 2
    with torch.cuda.stream(shard.stream):
        grad = torch.randn(shard.pooled_shape(w0.batch), generator=gen, device=device,
                           dtype=torch.float32).mul_(1e-3)
        if grad_dtype == "bfloat16":
            grad = grad.to(torch.bfloat16)  # round to nearest even, as the transport cast
        grad_out = None
        none_opt = None
        if w0.optimizer == "none":
            from flare_amd import _native

            grad_out = torch.empty((max(p.n for p in plans), w0.dim), dtype=torch.float32, device=device)
            none_opt = _native.FlareOptimizer()
            none_opt.kind = _native.OPT_NONE
    # unique counts of every batch (one dedup each, before timing)
    uniques = []
    for p in plans:
        p.dedup()
    shard.synchronize()
    for p in plans:
        uniques.append(int(p.unique_count.item()))
    log(f"setup {time.time() - t_setup:.1f}s: N={[p.n for p in plans][:3]}..., U={uniques[:3]}...")

    if args.copy_mib > 0:
        src = torch.ones(args.copy_mib << 18, dtype=torch.float32, device=device)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"copy calibration: 3 x {args.copy_mib} MiB read + {args.copy_mib} MiB written")
        del src, dst

    pipelined = args.order == "pipelined" and not args.overlap
    if pipelined and len(plans) < 2:
        raise SystemExit("the pipelined order needs at least 2 batches (the next batch's dedup runs beside "
                         "the current batch's update, each in its own workspace)")
    stream = shard.stream
    aux = torch.cuda.Stream(device=device)  # --overlap: the dedup beside the forward

    pipe = PooledStepPipeline(plans) if pipelined else None

    def run(i):
        if pipelined:
            pipe.step(i, grad, grad_out=grad_out, optimizer=none_opt)
        else:
            p = plans[i % len(plans)]
            p.forward()
            p.dedup()
            p.apply(grad, grad_out=grad_out, optimizer=none_opt)

    # every call below is enqueued with the shard's stream current, so the plans order nothing
    stream_ctx = torch.cuda.stream(stream)
    stream_ctx.__enter__()
    for i in range(args.warmup):
        run(i)
    shard.synchronize()
    torch.cuda.synchronize()

    overlap = args.overlap
    events = [[torch.cuda.Event(enable_timing=True) for _ in range(7)] for _ in range(args.steps)]
    # markers inside the update call, after sums_kernel and after the folds (recorded once
    # here so that each event exists before its handle is taken).  The update call launches
    # nothing before sums_kernel or after apply_kernel, so ev[4] and ev[5] bound those two.
    # Each record is a marker packet of a few microseconds on the stream, so none is
    # recorded twice at one point.
    markers = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(args.steps)]
    for mk in markers:
        for e in mk:
            e.record(stream)
    handles = [(ctypes.c_void_p * 4)(None, mk[0].cuda_event, mk[1].cuda_event, None) for mk in markers]
    lib = _native.library()
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    order = []
    fwd_start = [ev[0] for ev in events]  # the event before each step's forward
    for i in range(args.steps):
        k = (args.warmup + i) % len(plans)
        p = plans[k]
        order.append(k)
        ev = events[i]
        ev[0].record(stream)
        if pipelined:
            # PooledStepPipeline: forward; then this batch's update (its dedup ran beside the
            # previous update) while the next batch's dedup runs on the pipeline's stream.  A step
            # lasts from its forward to the next step's forward; the last one ends when the final
            # dedup is done.  Only the step boundaries and the end of the forward are marked here
            # (each mark is a marker packet on the stream); the update and dedup phases are timed
            # in an instrumented pass after this one.
            marks = {"forward_done": None}
            pipe.step(args.warmup + i, grad, grad_out=grad_out, optimizer=none_opt, marks=marks)
            ev[1] = marks["forward_done"]
            if i > 0:
                events[i - 1][6] = ev[0]
            if i + 1 == args.steps:
                pipe.finish()
                ev[6].record(stream)
            continue
        if overlap:
            # dedup (ids only) on a second stream, concurrent with the forward
            aux.wait_stream(stream)
            ev[2].record(aux)
            p._dedup_on(int(aux.cuda_stream))
            ev[3].record(aux)
            p.forward()
            ev[1].record(stream)
            stream.wait_event(ev[3])
        elif args.order == "dedup-first":
            ev[2] = ev[0]
            p.dedup()
            ev[3].record(stream)
            fwd_start[i] = ev[3]
            p.forward()  # one launch: the pooled gather kernel
            ev[1].record(stream)
        else:
            p.forward()
            ev[1].record(stream)
            ev[2] = ev[1]
            p.dedup()
            ev[3].record(stream)
        if overlap:
            ev[4].record(stream)
        else:
            ev[4] = ev[1] if args.order == "dedup-first" else ev[3]
        _native.check(lib.flare_set_update_events(ctypes.cast(handles[i], ctypes.c_void_p), 4))
        p.apply(grad, grad_out=grad_out, optimizer=none_opt)
        ev[5].record(stream)
    torch.cuda.synchronize()
    wall1 = time.perf_counter()
    # pipelined: the same steps again with every phase marked (the timing of the update's
    # kernels and of the dedup beside them; not part of the value)
    phase_events, phase_markers, phase_order = events, markers, order
    if pipelined:
        phase_events = [[None] * 7 for _ in range(args.steps)]
        phase_order = []
        for i in range(args.steps):
            k = (args.warmup + args.steps + i) % len(plans)
            phase_order.append(k)
            marks = dict.fromkeys(("forward_done", "update_start", "dedup_start", "dedup_done", "update_done"))
            _native.check(lib.flare_set_update_events(ctypes.cast(handles[i], ctypes.c_void_p), 4))
            pipe.step(args.warmup + args.steps + i, grad, grad_out=grad_out, optimizer=none_opt, marks=marks)
            ev = phase_events[i]
            ev[1], ev[2], ev[3], ev[4], ev[5] = (marks["forward_done"], marks["dedup_start"], marks["dedup_done"],
                                                 marks["update_start"], marks["update_done"])
        pipe.finish()
        torch.cuda.synchronize()
    stream_ctx.__exit__(None, None, None)
    _native.check(lib.flare_set_update_events(None, 0))
    timed_errors = int(lib.flare_take_device_errors(int(stream.cuda_stream)))
    check = {"timed_steps_device_errors": timed_errors}
    if not args.no_check:
        t_check = time.time()
        check.update(full_size_check(shard, plans[0], batches[0], grad, grad_out, none_opt))
        check["seconds"] = round(time.time() - t_check, 1)
        log(f"full-size check: {check}")
    check["passed"] = bool(timed_errors == 0 and check.get("passed", True))

    kernel_bytes = [update_kernel_bytes(b, s, g_bytes) for b in batches]
    step_ms, fwd_ms, dedup_ms, apply_ms = [], [], [], []
    step_gbs, fwd_gbs, upd_gbs = [], [], []
    sums_ms, fold_ms, applyk_ms, sums_gbs, applyk_gbs = [], [], [], [], []
    for i, ev in enumerate(events):  # the timed steps: step and forward
        b = batches[order[i]]
        f = fwd_start[i].elapsed_time(ev[1])
        t = ev[0].elapsed_time(ev[6] if pipelined else ev[5])
        step_ms.append(t)
        fwd_ms.append(f)
        fb, bb, ub = step_bytes(b.num_ids, uniques[order[i]], b.batch, b.num_tables, b.dim, s,
                                b.weights is not None, b.optimizer, g_bytes)
        step_gbs.append((fb + bb) / (t * 1e-3) / 1e9)
        fwd_gbs.append(fb / (f * 1e-3) / 1e9)
    for i, ev in enumerate(phase_events):  # dedup and update (the timed steps, or the marked pass)
        b = batches[phase_order[i]]
        a = ev[4].elapsed_time(ev[5])
        dedup_ms.append(ev[2].elapsed_time(ev[3]))
        apply_ms.append(a)
        fb, bb, ub = step_bytes(b.num_ids, uniques[phase_order[i]], b.batch, b.num_tables, b.dim, s,
                                b.weights is not None, b.optimizer, g_bytes)
        upd_gbs.append(ub / (a * 1e-3) / 1e9)
        mk = phase_markers[i]
        sm, fm, am = ev[4].elapsed_time(mk[0]), mk[0].elapsed_time(mk[1]), mk[1].elapsed_time(ev[5])
        sums_ms.append(sm)
        fold_ms.append(fm)
        applyk_ms.append(am)
        sb, ab = kernel_bytes[phase_order[i]]
        sums_gbs.append(sb / (sm * 1e-3) / 1e9)
        applyk_gbs.append(ab / (am * 1e-3) / 1e9)
    med = statistics.median(step_ms)
    rows = w0.batch * w0.num_tables
    achieved_step = statistics.median(step_gbs)
    fb0, bb0, ub0 = step_bytes(w0.num_ids, uniques[0], w0.batch, w0.num_tables, w0.dim, s,
                               w0.weights is not None, w0.optimizer, g_bytes)
    sb0, ab0 = kernel_bytes[0]

    def roofline(kernel, what, gbs, ms, nbytes):
        return {"kernel": f"{kernel} ({what})", "bound": "hbm", "achieved": statistics.median(gbs),
                "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": statistics.median(gbs) / PEAK_HBM_GBS,
                "traffic": kernel_traffic(config, kernel), "algorithmic_bytes_per_launch": nbytes,
                "kernel_ms": statistics.median(ms)}

    if w0.optimizer == "none":
        sums_name = ("sums_kernel", "segment sums of long keys; one launch per step")
        apply_name = ("apply_kernel", "short-key sums and the reduced gradients; one launch per step")
    else:
        sums_name = ("piece_sums_kernel", "per-piece sums of keys with several occurrences; one launch per step")
        apply_name = ("key_apply_kernel", "row-wise update of every key; one launch per step")
    # the forward kernel the library picks for this batch: one id per bag (table-major plan),
    # bags of at most 2 ids on average, or the general pooled gather
    if plans[0]._dedup_layout & _native.LAYOUT_ONE_ID_PER_BAG:
        fwd_name = ("pooled_one_kernel", "CSR pooled gather of one id per bag, forward; one launch per step")
    elif w0.num_ids <= 2 * w0.batch * w0.num_tables:
        fwd_name = ("pooled_short_kernel", "CSR pooled gather of short bags, forward; one launch per step")
    else:
        fwd_name = ("pooled_kernel", "CSR pooled gather, forward; one launch per step")
    kernels = [roofline(*fwd_name, fwd_gbs, fwd_ms, fb0),
               roofline(*sums_name, sums_gbs, sums_ms, sb0),
               roofline(*apply_name, applyk_gbs, applyk_ms, ab0)]
    dominant = max(kernels, key=lambda k: k["kernel_ms"])
    result = {
        "metric": METRIC,
        "value": rows / (med * 1e-3),
        "unit": "pooled rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": med,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": f"f32 ({'bf16' if w0.value_dtype == 'bfloat16' else w0.value_dtype} rows, "
                 f"{'bf16' if grad_dtype == 'bfloat16' else 'f32'} pooled grads)",
        "data": "synthetic (seeded Zipf ids, N(0,1e-3) pooled grads, U(-0.01,0.01) rows)",
        "config": {
            "workload": WORKLOAD_NAMES[config],
            "workload_id": config,
            "tables": w0.num_tables,
            "batch": w0.batch,
            "dim": w0.dim,
            "ids_per_step": w0.num_ids,
            "unique_per_step": uniques[0],
            "rotated_batches": len(plans),
            "dedup": "concurrent with the forward" if overlap else
                     ("one batch ahead: the next batch's dedup on a second stream beside this batch's "
                      "update; each step ends when both are done" if pipelined else
                      ("before the forward, same stream" if args.order == "dedup-first" else
                       "after the forward, same stream")),
            "pooled_layout": "[T, B, D]" if args.layout == "table_major" else "[B, T, D]",
            "pooled_grad_dtype": grad_dtype,
        },
        "hbm_gbs": achieved_step,
        "hbm_frac": achieved_step / PEAK_HBM_GBS,
        "algorithmic_bytes_per_step": fb0 + bb0,
        "phases_source": (f"step and forward: the timed steps; dedup and update phases: {args.steps} further steps "
                          "with every phase marked (the timed steps mark only step boundaries and the forward)"
                          if pipelined else "the timed steps"),
        "phases_ms": {
            "forward_pooled_gather": statistics.median(fwd_ms),
            "dedup_sort_unique": statistics.median(dedup_ms),
            "segment_reduce_update": statistics.median(apply_ms),
            "update_sums_kernel": statistics.median(sums_ms),
            "update_folds": statistics.median(fold_ms),
            "update_apply_kernel": statistics.median(applyk_ms),
        },
        "phases_gbs": {
            "forward_pooled_gather": statistics.median(fwd_gbs),
            "segment_reduce_update": statistics.median(upd_gbs),
        },
        "wall_ms_per_step": (wall1 - wall0) * 1e3 / args.steps,
        "roofline": dominant,
        "roofline_kernels": kernels,
        "cpu_baseline": None,
        "check": check,
    }
    if not args.no_cpu_baseline:
        del plans, grad
        torch.cuda.empty_cache()
        try:
            result["cpu_baseline"] = cpu_baseline(config, args.cpu_seconds)
        except Exception as error:  # the GPU result stands without the baseline
            log(f"cpu baseline failed: {error!r}")
    print(json.dumps(result), flush=True)
    if not check["passed"]:
        log("the full-size correctness check failed: the measured step is not valid")
        return 1
    return 0


if __name__ == "__main__":
    sys.exit(main())
