"""The C-ABI library (CPU only: no kernel is launched).

Checks that ``libflare_amd.so`` loads, exports every function that
``include/flare_amd.h`` declares, and that argument validation, which runs on
the host before any device work, returns the documented status codes.
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from flare_amd import _native

HEADER = Path(__file__).resolve().parents[1] / "include" / "flare_amd.h"


def declared_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(flare_[a-z_0-9]+)\s*\(", text)))


def test_header_declares_the_boundary():
    names = declared_functions()
    for required in ("flare_gather", "flare_gather_pooled", "flare_gather_pooled_csr", "flare_scatter",
                     "flare_scatter_pooled", "flare_unique_first_occurrence", "flare_sparse_update",
                     "flare_pooled_backward", "flare_last_error"):
        assert required in names


def test_library_exports_every_declared_symbol():
    lib = _native.library()
    missing = [name for name in declared_functions() if not hasattr(lib, name)]
    assert not missing, missing
    assert set(_native.SIGNATURES) == set(declared_functions())


def test_abi_version_matches_header():
    version = int(re.search(r"#define FLARE_ABI_VERSION (\d+)", HEADER.read_text()).group(1))
    assert _native.library().flare_abi_version() == version


def test_workspace_sizes_are_host_arithmetic():
    lib = _native.library()
    small = lib.flare_pooled_backward_workspace_bytes(1000, 10**6, 128)
    large = lib.flare_pooled_backward_workspace_bytes(1_703_936, 23_000_000, 128)
    # per-key fp32 gradient sums (n x dim) plus sort / run bookkeeping
    assert 0 < small < large < 1_703_936 * 128 * 4 + 256 * 2**20
    assert lib.flare_unique_workspace_bytes(10, _native.INT64) > 0
    assert lib.flare_scatter_workspace_bytes(0, 4, 3) > 0


def _call(name, *args):
    return getattr(_native.library(), name)(*args)


def test_dtype_errors_map_to_type_error():
    status = _call("flare_gather", None, 99, 4, 3, None, 4, 4, None, None)
    assert status == _native.ERR_DTYPE
    with pytest.raises(TypeError, match="float16, bfloat16 or float32"):
        _native.check(status)
    status = _call("flare_unique_first_occurrence", None, _native.FLOAT32, 3, 0, None, None, None,
                   None, None, 0, None)
    with pytest.raises(TypeError, match="integer keys"):
        _native.check(status)


def test_width_and_slot_errors_map_to_value_error():
    status = _call("flare_gather_pooled", None, _native.FLOAT32, 4, 3, None, 4, 0, 2, 4, 0, None, None, None)
    assert status == _native.ERR_WIDTH
    with pytest.raises(ValueError, match="positive target widths"):
        _native.check(status)
    status = _call("flare_scatter_pooled", 2, 2, None, 3, 2, None, 1, 1, 2, None, None, 0, None)
    assert status == _native.ERR_SHAPE
    with pytest.raises(ValueError, match="inverse slots must match"):
        _native.check(status)


def test_optimizer_validation_on_host():
    opt = _native.FlareOptimizer()
    opt.kind = _native.OPT_ADAM
    opt.weight_decay = 0.1
    status = _call("flare_sparse_update", None, _native.FLOAT32, 10, 4, None, None, None,
                   ctypes.byref(opt), None, 1, None, 1, None, 0, None)
    assert status == _native.ERR_ARGUMENT and "weight_decay" in _native.last_error()
    opt.weight_decay = 0.0
    status = _call("flare_sparse_update", None, _native.FLOAT32, 10, 4, None, None, None,
                   ctypes.byref(opt), None, 1, None, 1, None, 0, None)
    assert status == _native.ERR_ARGUMENT and "Adam requires" in _native.last_error()
    status = _call("flare_sparse_update", None, _native.FLOAT32, 10, 4, None, None, None,
                   ctypes.byref(opt), None, 1, None, 0, None, 0, None)
    assert status == _native.ERR_ARGUMENT and "normalization_steps" in _native.last_error()


def test_status_mapping():
    with pytest.raises(RuntimeError):
        _native.check(_native.ERR_HIP)
    for code in (_native.ERR_SHAPE, _native.ERR_WIDTH, _native.ERR_ARGUMENT, _native.ERR_WORKSPACE, _native.ERR_LIMIT):
        with pytest.raises(ValueError):
            _native.check(code)
    _native.check(_native.OK)


def test_keymap_and_ingest_validation_on_host():
    lib = _native.library()
    assert lib.flare_keymap_bytes(63) == 0 and lib.flare_keymap_bytes(100) == 0
    assert lib.flare_keymap_bytes(64) == 256 + 64 * 16
    assert lib.flare_keymap_bytes(1 << 31) == 0
    assert lib.flare_keymap_workspace_bytes(-1) == 0 and lib.flare_keymap_workspace_bytes(10) > 0
    assert lib.flare_keymap_export_workspace_bytes(128) > 0
    status = _call("flare_keymap_init", None, 100, None)
    assert status == _native.ERR_ARGUMENT and "power of two" in _native.last_error()
    status = _call("flare_keymap_lookup_or_insert", None, 64, None, 4, 1, None, _native.FLOAT32, 10, 8,
                   0.0, 1.0, 0, None, None, None, 0, None)
    assert status == _native.ERR_ARGUMENT  # null map
    status = _call("flare_nested_global_positions", None, 3, 0, None, None, None, 0, None, None, None)
    assert status == _native.ERR_ARGUMENT and "nested levels" in _native.last_error()
    status = _call("flare_copy_rows", None, 4, None, 4, 3, None, None, 1, None)
    assert status == _native.ERR_SHAPE


def test_gradient_transport_dtype_validation_on_host():
    opt = _native.FlareOptimizer()
    opt.kind = _native.OPT_SGD
    status = _call("flare_sparse_update_ex", None, _native.FLOAT32, 10, 4, None, None, None, ctypes.byref(opt),
                   None, 1, None, _native.FLOAT16, 0, None, 1, None, 0, None)
    assert status == _native.ERR_DTYPE and "gradient_transport_dtype" in _native.last_error()
    with pytest.raises(TypeError, match="gradient_transport_dtype"):
        _native.check(status)
    status = _call("flare_check_finite", None, _native.FLOAT32, -1, None, None)
    assert status == _native.ERR_SHAPE


def test_update_event_markers_validation_on_host():
    assert _call("flare_set_update_events", None, 5) == _native.ERR_ARGUMENT
    assert "count must be 0..4" in _native.last_error()
    assert _call("flare_set_update_events", None, 2) == _native.ERR_ARGUMENT
    nulls = (ctypes.c_void_p * 2)(None, None)  # null entries: no marker at those points
    assert _call("flare_set_update_events", ctypes.cast(nulls, ctypes.c_void_p), 2) == _native.OK
    assert _call("flare_set_update_events", None, 0) == _native.OK


def test_stream_and_zero_fill_validation_on_host():
    assert _call("flare_zero_bytes", None, -1, None) == _native.ERR_SHAPE
    assert _call("flare_zero_bytes", None, 0, None) == _native.OK  # nothing to do, no launch
    assert _call("flare_zero_bytes", None, 8, None) == _native.ERR_ARGUMENT
    assert _call("flare_stream_create", None) == _native.ERR_ARGUMENT
    assert _call("flare_stream_destroy", None) == _native.ERR_ARGUMENT
    assert "null (default) stream" in _native.last_error()


def test_misaligned_workspace_is_refused_on_host():
    """The backward workspace is laid out from its first byte and used with 16-byte vectors:
    a misaligned one is refused before any launch (ValueError, FLARE_ERR_WORKSPACE)."""
    lib = _native.library()
    n, rows, dim = 1000, 5000, 64
    nbytes = lib.flare_pooled_backward_workspace_bytes(n, rows, dim)
    fake = 1 << 40  # never dereferenced: validation fails first
    with pytest.raises(ValueError, match="16-byte aligned"):
        _native.call("flare_pooled_dedup", fake, _native.INT64, n, fake, 1, n, fake, rows, dim, 0,
                     _native.LAYOUT_TABLE_MAJOR, None, None, None, fake + 8, nbytes, None)
    with pytest.raises(ValueError, match="smaller than"):
        _native.call("flare_pooled_dedup", fake, _native.INT64, n, fake, 1, n, fake, rows, dim, 0,
                     _native.LAYOUT_TABLE_MAJOR, None, None, None, fake, nbytes - 1, None)
