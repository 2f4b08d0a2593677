"""GPU parity of the HIP operator against the oracle and the reference's own vectors.

Mirrors tests/kernels/test_sparse_embedding_backend.py of the reference
(known answers at :78-89, :144-183, :225-233; duplicate-key scatter at
:353-390; slot-mismatch error at :393-407) and
tests/training/test_cupy_sparse_gradient_stream.py:24-76 (exact counts).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import sparse_oracle as O

pytestmark = pytest.mark.gpu


def _op(value_dtype="float32"):
    from flare_amd.operator import HipSparseEmbeddingOperator

    return HipSparseEmbeddingOperator(value_dtype, "float32", empty_cache=False)


def _host(t) -> np.ndarray:
    """Host copy of a torch tensor or of the operator's DeviceArray (bf16 as raw bits)."""
    from flare_amd.array import DeviceArray

    if isinstance(t, DeviceArray):
        t = t.tensor
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).cpu().numpy().view(np.uint16)
    return t.cpu().numpy()


def _dev_storage(arr: np.ndarray, storage: str, device) -> torch.Tensor:
    if storage == "bfloat16":
        return torch.from_numpy(arr.view(np.int16)).to(device).view(torch.bfloat16)
    return torch.from_numpy(np.ascontiguousarray(arr)).to(device)


def test_prewarm_probe(gpu_device, no_device_errors):
    op = _op()
    op.prewarm()
    no_device_errors()


def test_pooled_gather_known_answer(gpu_device, no_device_errors):
    # test_sparse_embedding_backend.py:78-89
    op = _op()
    emb = torch.arange(8, dtype=torch.float32, device=gpu_device).reshape(4, 2)
    inv = torch.tensor([0, 4, 2, 1], dtype=torch.int32, device=gpu_device)
    out = op.gather_pooled(emb, inv, 4, 2, (1, 1), 4)
    op.stream.synchronize()
    np.testing.assert_array_equal(_host(out).reshape(4, 2),
                                  [[0.0, 1.0], [0.0, 0.0], [4.0, 5.0], [2.0, 3.0]])
    no_device_errors()


def test_fp16_pooled_gather_known_answers(gpu_device, no_device_errors):
    op = _op("float16")
    # :162-172
    emb = torch.tensor([[1.5, 2.0], [3.0, 4.0]], dtype=torch.float16, device=gpu_device)
    out = op.gather_pooled(emb, np.asarray([0, 1, 2, 2], np.int32), 2, 2, (1, 2), 2)
    op.stream.synchronize()
    assert out.dtype == np.float16
    np.testing.assert_array_equal(_host(out), np.asarray([[[4.5, 6.0]], [[0.0, 0.0]]], np.float16))
    # :175-183 wide accumulation: 40000 - 40000 + 1 -> 1
    emb = torch.tensor([[40000.0], [-40000.0], [1.0]], dtype=torch.float16, device=gpu_device)
    out = op.gather_pooled(emb, np.asarray([0, 1, 2], np.int32), 1, 1, (1, 3), 3)
    op.stream.synchronize()
    np.testing.assert_array_equal(_host(out), np.asarray([[[1.0]]], np.float16))
    # :225-233 overflow to inf
    emb = torch.tensor([[65504.0], [65504.0]], dtype=torch.float16, device=gpu_device)
    out = op.gather_pooled(emb, np.asarray([0, 1], np.int32), 1, 1, (1, 2), 2)
    op.stream.synchronize()
    assert np.isinf(_host(out)).all()
    no_device_errors()


def test_empty_inputs_return_shapes_without_launch(gpu_device):
    op = _op("float16")
    emb = torch.empty((0, 2), dtype=torch.float16, device=gpu_device)
    inv = torch.empty((0,), dtype=torch.int32, device=gpu_device)
    assert tuple(op.gather_pooled(emb, inv, 0, 2, (1, 2), 0).shape) == (0, 1, 2)
    g = op.gather(emb, inv, 0, 2, 0)
    assert tuple(g.shape) == (0, 0, 2) and g.dtype == np.float16


@pytest.mark.parametrize("storage", ["float32", "float16", "bfloat16"])
@pytest.mark.parametrize("dim", [3, 8, 64, 128, 130])
def test_gather_matches_oracle_bitwise(gpu_device, no_device_errors, storage, dim):
    rng = np.random.default_rng(dim)
    rows = 97
    emb32 = rng.standard_normal((rows, dim), dtype=np.float32)
    emb = O.f32_to_storage(emb32, storage)
    inv = rng.integers(0, rows + 1, 301).astype(np.int32)
    op = _op(storage)
    out = op.gather(_dev_storage(emb, storage, gpu_device), inv, 7, dim, rows)
    op.stream.synchronize()
    exp = O.gather(emb, inv, 7, dim, rows)
    np.testing.assert_array_equal(_host(out), exp)
    no_device_errors()


@pytest.mark.parametrize("storage", ["float32", "float16", "bfloat16"])
@pytest.mark.parametrize("pooling", ["sum", "mean", "weighted"])
@pytest.mark.parametrize("shape", [(5, 3, 7, 3), (16, 2, 30, 128), (9, 4, 1, 64), (3, 1, 65, 40), (4, 2, 3, 418)])
def test_gather_pooled_matches_oracle_bitwise(gpu_device, no_device_errors, storage, pooling, shape):
    batch, features, max_el, dim = shape
    rng = np.random.default_rng(batch * 1000 + dim)
    rows = 50
    emb = O.f32_to_storage(rng.standard_normal((rows, dim), dtype=np.float32), storage)
    inv = rng.integers(0, rows, (batch, features, max_el)).astype(np.int32)
    inv[rng.random(inv.shape) < 0.3] = rows
    weights = rng.random(inv.shape, dtype=np.float32)
    op = _op(storage)
    out = op.gather_pooled(_dev_storage(emb, storage, gpu_device), inv, batch, dim, (features, max_el), rows,
                           pooling=pooling, per_sample_weights=weights if pooling == "weighted" else None)
    op.stream.synchronize()
    exp = O.gather_pooled(emb, inv, batch, dim, (features, max_el), rows, storage=storage,
                          pooling=pooling, weights=weights)
    np.testing.assert_array_equal(_host(out), exp)
    no_device_errors()


@pytest.mark.parametrize("feature_count,max_elements,dim", [(12, 30, 128), (44, 30, 40), (2, 1, 418)])
def test_scatter_pooled_matches_duplicate_key_sum(gpu_device, no_device_errors, feature_count, max_elements, dim):
    # reference test_sparse_embedding_backend.py:353-390 (seed 93, 80% pad, tol 2e-4)
    batch_size, rows = 48, 256
    rng = np.random.default_rng(93)
    inverse = rng.integers(0, rows // 4, (batch_size, feature_count, max_elements), dtype=np.int32)
    inverse[rng.random(inverse.shape) < 0.8] = rows
    gradient = rng.standard_normal((batch_size, feature_count, dim)).astype(np.float32)
    flat_inverse = inverse.reshape(-1)
    flat_gradient = np.repeat(gradient.reshape(-1, dim), max_elements, axis=0)
    valid = flat_inverse != rows
    expected = np.zeros((rows, dim), dtype=np.float32)
    np.add.at(expected, flat_inverse[valid], flat_gradient[valid])
    op = _op("float16")
    actual = op.scatter_pooled(rows, dim, torch.from_numpy(inverse).to(gpu_device), rows,
                               torch.from_numpy(gradient).to(gpu_device), (feature_count, max_elements))
    op.stream.synchronize()
    got = _host(actual)
    np.testing.assert_allclose(got, expected, atol=2e-4, rtol=2e-4)
    # bit-exact against the oracle's (documented) reduction order
    exact = O.scatter_pooled(rows, dim, inverse, rows, gradient, (feature_count, max_elements))
    np.testing.assert_array_equal(got, exact)
    no_device_errors()


def test_pooled_scatter_rejects_partial_inverse_slots(gpu_device):
    # reference :393-407
    op = _op("float16")
    with pytest.raises(ValueError, match="inverse slots must match"):
        op.scatter_pooled(2, 2, torch.tensor([0, 1, 2], dtype=torch.int32, device=gpu_device), 2,
                          torch.ones((1, 1, 2), dtype=torch.float32, device=gpu_device), (1, 2))


def test_scatter_exact_counts(gpu_device, no_device_errors):
    # tests/training/test_cupy_sparse_gradient_stream.py:24-76: grads 1/(256*2^i)
    # sum exactly to count/(256*2^i) in fp32
    batch_size, feature_count, max_elements, width, rows = 2560, 4, 4, 32, 512
    rng = np.random.default_rng(13)
    inverse = rng.integers(0, rows + 1, (batch_size, feature_count, max_elements), dtype=np.int32)
    counts = np.bincount(inverse[inverse != rows], minlength=rows)
    op = _op("float16")
    for index in range(3):
        grad = torch.full((batch_size, feature_count, width), 1 / (256 * (2 ** index)),
                          dtype=torch.bfloat16, device=gpu_device).to(torch.float32)
        out = op.scatter_pooled(rows, width, torch.from_numpy(inverse).to(gpu_device), rows, grad,
                                (feature_count, max_elements))
        op.stream.synchronize()
        expected = np.broadcast_to((counts / (256 * (2 ** index)))[:, None], (rows, width))
        np.testing.assert_array_equal(_host(out), expected)
        np.testing.assert_array_equal(_host(out.astype("bfloat16").astype("float32")), expected)
    no_device_errors()


@pytest.mark.parametrize("slots,rows,dim,seed", [(8, 4, 3, 0), (5000, 17, 4, 1), (20000, 3000, 33, 2), (70000, 50, 128, 3)])
def test_scatter_matches_oracle(gpu_device, no_device_errors, slots, rows, dim, seed):
    rng = np.random.default_rng(seed)
    inv = rng.integers(0, rows + 1, slots).astype(np.int32)
    grad = rng.standard_normal((slots, dim), dtype=np.float32)
    op = _op()
    out = op.scatter(rows, dim, torch.from_numpy(inv).to(gpu_device), rows, torch.from_numpy(grad).to(gpu_device))
    op.stream.synchronize()
    got = _host(out)
    np.testing.assert_array_equal(got, O.scatter(rows, dim, inv, rows, grad))
    # and within tolerance of plain slot-order (Numba reference order) sums
    ref = O.scatter(rows, dim, inv, rows, grad, unit=max(slots, 1))
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5 * np.sqrt(slots / rows))
    no_device_errors()


def test_gather_out_of_range_ids_are_zero_and_flagged(gpu_device, no_device_errors):
    op = _op()
    emb = torch.ones((4, 2), dtype=torch.float32, device=gpu_device)
    out = op.gather(emb, torch.tensor([0, 9, -3, 4], dtype=torch.int32, device=gpu_device), 4, 2, 4)
    op.stream.synchronize()
    np.testing.assert_array_equal(_host(out).reshape(4, 2), [[1, 1], [0, 0], [0, 0], [0, 0]])
    no_device_errors(expected=1)


@pytest.mark.parametrize("dim", [128, 512, 1024, 2048])
def test_scatter_hot_key_across_many_units_bit_exact(gpu_device, no_device_errors, dim):
    """A key with thousands of occurrences (its unit partials folded by one block) at every row width."""
    op = _op()
    rng = np.random.default_rng(dim)
    rows, slots = 50, 3000
    inverse = rng.integers(0, rows + 1, slots).astype(np.int32)  # rows == pad
    inverse[rng.random(slots) < 0.5] = 7                          # hot key: ~1500 occurrences, ~24 units
    grad = rng.standard_normal((slots, dim)).astype(np.float32)
    out = op.scatter(rows, dim, torch.from_numpy(inverse).to(gpu_device), rows,
                     torch.from_numpy(grad).to(gpu_device))
    op.stream.synchronize()
    np.testing.assert_array_equal(_host(out), O.scatter(rows, dim, inverse, rows, grad))
    no_device_errors()


@pytest.mark.parametrize("dim", [4, 128, 300, 2048])
def test_scatter_key_past_the_fold_chunk_bit_exact(gpu_device, no_device_errors, dim):
    """Keys spanning more than 64 units (two-level fold: runs of 64 unit partials folded in
    parallel, then the runs) and one spanning exactly 64, against the oracle bit for bit."""
    op = _op()
    rng = np.random.default_rng(500 + dim)
    rows = 40
    slots = 64 * 64 * 3 + 777
    inverse = rng.integers(0, rows + 1, slots).astype(np.int32)  # rows == pad
    pick = rng.random(slots)
    inverse[pick < 0.55] = 3        # ~6.9K occurrences: ~110 units
    inverse[(pick >= 0.55) & (pick < 0.85)] = 11
    grad = rng.standard_normal((slots, dim)).astype(np.float32)
    out = op.scatter(rows, dim, torch.from_numpy(inverse).to(gpu_device), rows,
                     torch.from_numpy(grad).to(gpu_device))
    op.stream.synchronize()
    np.testing.assert_array_equal(_host(out), O.scatter(rows, dim, inverse, rows, grad))
    # exactly 64 units for one key: the one-level fold
    inv2 = np.full(64 * 64, 5, np.int32)
    g2 = rng.standard_normal((inv2.size, dim)).astype(np.float32)
    out2 = op.scatter(rows, dim, torch.from_numpy(inv2).to(gpu_device), rows, torch.from_numpy(g2).to(gpu_device))
    op.stream.synchronize()
    np.testing.assert_array_equal(_host(out2), O.scatter(rows, dim, inv2, rows, g2))
    no_device_errors()
