"""Host-side drop-in contract: the names, arguments and array protocol the reference's
unchanged callers use, replayed on the CPU.

- ``sparse_embedding`` as ``DynamicSparseEmbeddingSPMD`` imports and configures it
  (``src/flare/runtime/fluxway/workers/dynamic_embedding.py:6-10,69-106,250-276``);
- the array protocol of the operator's results as ``scatter_sparse_grads`` and
  ``materialize_recsys_sparse_inputs`` use it
  (``recipes/recsys/ranking/workers/train_worker.py:488-530``,
  ``recipes/recsys/ranking/schema/materialization.py:41-53``);
- DLPack capsules in (``prepare_dlpack_input``, ``dynamic_embedding.py:396-400,514``);
- the precision contract's dispatch over numpy / device / torch arrays
  (``src/flare/runtime/sparse_precision.py:98-192``).
"""

from __future__ import annotations

import importlib
import sys

import numpy as np
import pytest
import torch

from flare_amd.array import BFLOAT16, DeviceArray, dtype_name
from flare_amd.conversion import is_dlpack_capsule, to_device
from flare_amd.precision import (
    prepare_sparse_native_gradient,
    require_finite_sparse_values,
    require_sparse_key_dtype,
    require_sparse_tensor_dtype,
)


@pytest.fixture()
def se():
    """``import sparse_embedding as se`` resolving to this package's store surface."""
    saved = {k: sys.modules.get(k) for k in ("sparse_embedding", "sparse_embedding.checkpoint")}
    import flare_amd.sparse_embedding as facade

    facade.install()
    module = importlib.import_module("sparse_embedding")
    yield module
    for k, v in saved.items():
        if v is None:
            sys.modules.pop(k, None)
        else:
            sys.modules[k] = v


def _create_sparse_optimizer(se, kind, policy="constant", **kw):
    """The worker's create_sparse_optimizer (dynamic_embedding.py:69-106), restated."""
    policy_factories = {
        "constant": se.ConstantLrPolicy,
        "sqrt_decay": se.SqrtDecayLrPolicy,
        "log_decay": se.LogDecayLrPolicy,
        "inverse_decay": se.InverseDecayLrPolicy,
        "cosine_frequency": lambda: se.CosineFrequencyLrPolicy(min_lr_ratio=0.1, max_score=10.0),
        "custom_lut": lambda: se.CustomLutLrPolicy(lut=[1.0]),
    }
    dynamic_lr_policy = policy_factories[policy]()
    if kind == "adam":
        return se.Adam(lr=kw.get("lr", 0.01), beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.0,
                       dynamic_lr_policy=dynamic_lr_policy)
    return se.Sgd(lr=kw.get("lr", 0.01), weight_decay=0.0, dynamic_lr_policy=dynamic_lr_policy)


def test_worker_imports_resolve(se):
    from sparse_embedding.checkpoint import SUPPORTED_KEY_DTYPES, CheckpointSaveMode, PartitionSpec

    assert {"int32", "uint32", "int64", "uint64"} == set(SUPPORTED_KEY_DTYPES)
    assert PartitionSpec.modulo() != PartitionSpec.hash()
    assert CheckpointSaveMode.INCREMENTAL != CheckpointSaveMode.FULL
    for name in ("EmbeddingConfig", "EmbeddingStore", "Uniform", "Adam", "Sgd", "AutoStorage",
                 "StorageTuningOptions", "Optimizer", "ConstantLrPolicy"):
        assert hasattr(se, name), name


@pytest.mark.parametrize("kind", ["adam", "sgd"])
@pytest.mark.parametrize("policy", ["constant", "sqrt_decay", "custom_lut"])
def test_worker_optimizer_configs(se, kind, policy):
    opt = _create_sparse_optimizer(se, kind, policy)
    assert isinstance(opt, se.Optimizer)
    if policy == "constant":
        native = opt._native()
        assert native.dynamic_lr_policy == "constant"
    else:
        # only the constant policy is implemented: the store refuses the others
        from flare_amd.store import _native_optimizer

        with pytest.raises(ValueError, match="learning-rate policy"):
            _native_optimizer(opt._native())


def test_embedding_config_as_the_worker_fills_it(se):
    cfg = se.EmbeddingConfig(
        dims=[16, 32], thread_budget=4, value_dtype="float16", gradient_dtype="float32",
        optimizer_dtype="float32", key_dtype="int64",
        storage=se.AutoStorage(memory_limit_bytes=None, spill_directory=None, max_spill_bytes=None),
        enable_optimizer=True,
    )
    assert list(cfg.dims) == [16, 32] and cfg.value_dtype == "float16"
    if not torch.cuda.is_available():
        # the store lives in HBM: without a GPU it fails loudly instead of falling back
        with pytest.raises(RuntimeError):
            se.EmbeddingStore(embedding_config=cfg, initializer_config=se.Uniform(min_val=-0.01, max_val=0.01),
                              optimizer_config=_create_sparse_optimizer(se, "adam"), score_policy="lfu")


def test_store_rejects_unsupported_options(se):
    cfg = se.EmbeddingConfig(dims=[4], key_dtype="int64")
    with pytest.raises(ValueError, match="score_policy"):
        se.EmbeddingStore(embedding_config=cfg, optimizer_config=se.Sgd(lr=1.0), score_policy="lru")
    with pytest.raises(ValueError, match="key_dtype"):
        se.EmbeddingStore(embedding_config=se.EmbeddingConfig(dims=[4], key_dtype="float32"),
                          optimizer_config=se.Sgd(lr=1.0))
    with pytest.raises(ValueError, match="optimizer_config"):
        se.EmbeddingStore(embedding_config=cfg)


def test_device_array_protocol_on_host_tensors():
    """What scatter_sparse_grads and materialization do with an operator result
    (train_worker.py:514-522, materialization.py:41-53)."""
    grad = DeviceArray(torch.arange(6, dtype=torch.float32).reshape(3, 2))
    assert np.dtype(grad.dtype).name == "float32"
    assert grad.shape == (3, 2) and grad.ndim == 2 and grad.size == 6 and len(grad) == 3
    assert grad.strides == (8, 4) and grad.nbytes == 24
    half = grad.astype("float16")
    assert isinstance(half, DeviceArray) and np.dtype(half.dtype) == np.float16
    np.testing.assert_array_equal(np.asarray(half), np.arange(6, dtype=np.float16).reshape(3, 2))
    assert grad.astype("float32", copy=False) is grad
    assert int(grad[2, 1]) == 5 and float(grad[1][0]) == 2.0
    assert grad.reshape((-1,)).shape == (6,) and grad.reshape(2, 3).shape == (2, 3)
    counts = DeviceArray(torch.tensor([7], dtype=torch.int64))
    assert int(counts[0]) == 7 and counts[0].item() == 7
    assert [0, 1, 2, 3, 4, 5, 6, 7][counts[0]] == 7  # __index__
    np.testing.assert_array_equal(grad.get(), np.arange(6, dtype=np.float32).reshape(3, 2))
    # DLPack export of the wrapped tensor (the JAX binding consumes __dlpack__)
    back = torch.from_dlpack(grad)
    assert back.data_ptr() == grad.data_ptr()
    with pytest.raises(AttributeError):
        grad.__cuda_array_interface__  # host tensors have none


def test_bfloat16_dtype_name_without_ml_dtypes():
    t = DeviceArray(torch.zeros(3, dtype=torch.bfloat16))
    assert dtype_name(t.dtype) == "bfloat16"
    assert t.dtype == "bfloat16" or getattr(t.dtype, "name", None) == "bfloat16"
    assert BFLOAT16 == "bfloat16" and BFLOAT16.itemsize == 2
    require_sparse_tensor_dtype(t, "bfloat16", boundary="test")
    with pytest.raises(TypeError, match="mismatch"):
        require_sparse_tensor_dtype(t, "float32", boundary="test")


def test_dlpack_capsules_are_accepted():
    """prepare_dlpack_input(keys) hands the store a DLPack capsule (dynamic_embedding.py:396-400)."""
    keys = np.asarray([5, 3, 5], np.int64)
    capsule = keys.__dlpack__()
    assert is_dlpack_capsule(capsule)
    t = to_device(capsule, torch.device("cpu"))
    np.testing.assert_array_equal(t.numpy(), keys)
    legacy = torch.utils.dlpack.to_dlpack(torch.tensor([1.0, 2.0]))
    np.testing.assert_array_equal(to_device(legacy, torch.device("cpu")).numpy(), [1.0, 2.0])
    np.testing.assert_array_equal(to_device(DeviceArray(torch.tensor([4])), torch.device("cpu")).numpy(), [4])


def test_native_gradient_dispatch():
    """prepare_sparse_native_gradient over numpy, torch and device arrays
    (sparse_precision.py:150-192): transport dtype checked, cast to fp32, opt-in finite check."""
    g = np.ones((2, 3), np.float32)
    out = prepare_sparse_native_gradient(g, transport_dtype="float32", native_dtype="float32")
    assert isinstance(out, np.ndarray) and out.dtype == np.float32
    t = torch.ones(2, 3, dtype=torch.bfloat16)
    out = prepare_sparse_native_gradient(t, transport_dtype="bfloat16", native_dtype="float32")
    assert out.dtype == torch.float32
    out = prepare_sparse_native_gradient(DeviceArray(t), transport_dtype="bfloat16", native_dtype="float32")
    assert isinstance(out, DeviceArray) and dtype_name(out.dtype) == "float32"
    with pytest.raises(TypeError, match="transport dtype mismatch"):
        prepare_sparse_native_gradient(g, transport_dtype="bfloat16", native_dtype="float32")
    with pytest.raises(ValueError, match="gradient_dtype"):
        prepare_sparse_native_gradient(g, transport_dtype="float32", native_dtype="float16")
    with pytest.raises(FloatingPointError, match="sparse_native_gradient"):
        prepare_sparse_native_gradient(np.asarray([np.nan], np.float32), transport_dtype="float32",
                                       native_dtype="float32", validate_values=True)
    with pytest.raises(TypeError, match="unsupported sparse"):
        prepare_sparse_native_gradient([1.0], transport_dtype="float32", native_dtype="float32")
    with pytest.raises(FloatingPointError, match="at b"):
        require_finite_sparse_values(torch.tensor([np.inf]), "float32", boundary="b")


def test_key_dtype_contract():
    require_sparse_key_dtype(np.zeros(2, np.int64), "int64", boundary="lookup")
    with pytest.raises(TypeError, match="mismatch"):
        require_sparse_key_dtype(np.zeros(2, np.int32), "int64", boundary="lookup")
    with pytest.raises(TypeError, match="must be one of"):
        require_sparse_key_dtype(np.zeros(2, np.float32), "int64", boundary="lookup")
