"""Host arithmetic of bench.py's per-kernel algorithmic bytes (CPU only), on hand-counted cases."""

from __future__ import annotations

import sys
from pathlib import Path
from types import SimpleNamespace

import numpy as np

sys.path.insert(0, str(Path(__file__).resolve().parents[1]))
import bench  # noqa: E402


def _workload(keys, offsets, batch, tables, dim, optimizer):
    keys = np.asarray(keys, np.int64)
    return SimpleNamespace(global_keys=lambda: keys, offsets=np.asarray(offsets, np.int64), batch=batch,
                           num_tables=tables, dim=dim, optimizer=optimizer)


def test_pieces_singles_and_unit_crossing_keys_one_id_per_bag():
    # sorted positions: key 0 at 0..59 (one piece), key 1 at 60..61, key 2 at 62..64 (crosses
    # position 64: two pieces), key 3 at 65..66, key 4 at 67..69, key 5 once at 70 (single).
    # One id per bag, so every occurrence has its own gradient row.
    keys = [0] * 60 + [1] * 2 + [2] * 3 + [3] * 2 + [4] * 3 + [5]
    keys = np.random.default_rng(3).permutation(np.asarray(keys))  # order of occurrence is irrelevant
    w = _workload(keys, np.arange(72), 71, 1, 4, "rowwise_adagrad")
    sums, apply = bench.update_kernel_bytes(w, 2)
    n, n_multi, p_multi, u, n_single = 71, 70, 6, 6, 1
    assert sums == n_multi * 4 * 4 + n * 4 + p_multi * 4 * 4 + n * 4
    rows_state = 2 * u * 4 * 2 + 2 * u * 4
    assert apply == rows_state + n_single * 4 * 4 + p_multi * 4 * 4
    # bfloat16 pooled gradients: gradient rows at 2 bytes an element
    sums2, apply2 = bench.update_kernel_bytes(w, 2, 2)
    assert sums - sums2 == n_multi * 4 * 2 and apply - apply2 == n_single * 4 * 2


def test_a_bag_row_counts_once_per_kernel():
    # two bags of three ids: key 5 four times, keys 7 and 8 once each; piece_sums reads the two
    # bags' rows once (key 5 occurs in both), key_apply the single keys' bag row once
    w = _workload([5, 5, 5, 5, 7, 8], [0, 3, 6], 2, 1, 4, "sgd")
    sums, apply = bench.update_kernel_bytes(w, 4)
    assert sums == 2 * 4 * 4 + 6 * 4 + 1 * 4 * 4 + 6 * 4
    assert apply == 3 * (2 * 4 * 4) + 1 * 4 * 4 + 1 * 4 * 4


def test_reduced_gradient_kernels_long_and_short_keys():
    # optimizer "none" (reduced gradients): sums_kernel takes keys crossing a unit boundary or
    # of more than 4 positions, apply_kernel sums the others and writes U reduced rows
    keys = [0] * 60 + [1] * 2 + [2] * 3 + [3] * 2 + [4] * 3
    keys = np.random.default_rng(3).permutation(np.asarray(keys))
    w = _workload(keys, np.arange(71), 70, 1, 4, "none")
    sums, apply = bench.update_kernel_bytes(w, 2)
    n_long, p_long, u, u_long, n_short = 63, 3, 5, 2, 7
    assert sums == n_long * 4 * 4 + n_long * 4 + p_long * 4 * 4
    assert apply == u * 4 * 4 + n_short * 4 * 4 + n_short * 4 + u_long * 4 * 4


def test_step_bytes_follow_the_published_formula():
    # N ids, U unique rows, batch B, T tables, D, storage bytes s; weighted adds N*4 per phase
    n, u, b, t, d, s = 1000, 300, 64, 4, 16, 2
    fwd, bwd, upd = bench.step_bytes(n, u, b, t, d, s, True, "rowwise_adagrad")
    offsets = t * (b + 1) * 4
    assert fwd == n * 8 + offsets + n * 4 + u * d * s + b * t * d * s
    rows_state = 2 * u * d * s + 2 * u * 4
    assert bwd == n * 8 + offsets + n * 4 + b * t * d * 4 + u * 8 + n * 4 + rows_state
    assert upd == b * t * d * 4 + rows_state + n * 4
    # Adam: m and v rows plus a step counter per row; gradient-only: reduced rows out
    _, bwd_adam, _ = bench.step_bytes(n, u, b, t, d, s, False, "adam")
    assert bwd_adam == n * 8 + offsets + b * t * d * 4 + u * 8 + n * 4 + 2 * u * d * s + 2 * u * (2 * d * 4 + 4)
    _, bwd_none, _ = bench.step_bytes(n, u, b, t, d, s, False, "none")
    assert bwd_none == n * 8 + offsets + b * t * d * 4 + u * 8 + n * 4 + u * d * 4


def test_committed_traffic_covers_each_workloads_long_kernels():
    # roofline.traffic reads the committed counter runs: every workload needs its forward and its
    # two update kernels there, and each counter's copy calibration must be the one the counters
    # give on this GPU (FETCH_SIZE counts half of a copy's read bytes, WRITE_SIZE all written ones)
    expected = {1: ("pooled_kernel", "piece_sums_kernel", "key_apply_kernel"),
                2: ("pooled_one_kernel", "piece_sums_kernel", "key_apply_kernel"),
                3: ("pooled_kernel", "sums_kernel", "apply_kernel"),
                4: ("pooled_kernel", "piece_sums_kernel", "key_apply_kernel"),
                5: ("pooled_kernel", "piece_sums_kernel", "key_apply_kernel")}
    import json

    recs = json.loads((Path(bench.ROOT) / "profiles" / "step_kernel_traffic.json").read_text())["workloads"]
    for config, kernels in expected.items():
        rec = recs[str(config)]
        assert 1.9 < rec["fetch_scale"] < 2.1 and 0.95 < rec["write_scale"] < 1.05, config
        assert (Path(bench.ROOT) / rec["summary"]).exists(), config
        for k in kernels:
            traffic = bench.kernel_traffic(config, k)
            assert traffic is not None and traffic > 0, (config, k)
    assert bench.kernel_traffic(2, "no_such_kernel") is None
    assert bench.kernel_traffic(9, "pooled_kernel") is None
