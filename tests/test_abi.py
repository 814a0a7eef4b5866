"""The C-ABI library loads, exports every symbol include/helix_hip.h declares, and rejects bad
arguments on the host with the reference's TensorError variants — no GPU needed."""
import ctypes
import re
from pathlib import Path

import pytest

from helixml_amd import _ffi

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "helix_hip.h"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(hx_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_expected_entry_points():
    names = declared_functions()
    for must in ("hx_selective_scan_fwd", "hx_selective_state_update", "hx_s4_ref_fwd",
                 "hx_s4d_complex_fwd", "hx_linear_f32", "hx_matmul_f32", "hx_init", "hx_malloc",
                 "hx_free", "hx_last_error"):
        assert must in names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(_ffi.LIB_PATH))
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"


def test_binding_covers_header():
    assert set(declared_functions()) == set(_ffi.SIGNATURES)


def test_version():
    assert _ffi.lib().hx_version() >= 0x000100


@pytest.mark.parametrize("dstate", [0, 65])
def test_scan_rejects_dstate(dstate):
    rc = _ffi.lib().hx_selective_scan_fwd(1, 4, 4, dstate, 0, 1, *([None] * 11), None)
    assert rc == _ffi.UnsupportedOperation.status
    assert "dstate" in _ffi.last_error()
    with pytest.raises(_ffi.UnsupportedOperation):
        _ffi.check(rc)


def test_scan_rejects_dtype_and_negative_sizes():
    L = _ffi.lib()
    assert L.hx_selective_scan_fwd(1, 4, 4, 16, 7, 1, *([None] * 11), None) == _ffi.DTypeMismatch.status
    assert L.hx_selective_scan_fwd(-1, 4, 4, 16, 0, 1, *([None] * 11), None) == _ffi.InvalidDimension.status


def test_scan_empty_batch_is_noop():
    # batch == 0: nothing to do, no device call, OK
    assert _ffi.lib().hx_selective_scan_fwd(0, 4, 4, 16, 0, 1, *([None] * 11), None) == 0


def test_scan_null_pointers_rejected():
    rc = _ffi.lib().hx_selective_scan_fwd(1, 4, 4, 16, 0, 1, *([None] * 11), None)
    assert rc == _ffi.InvalidInput.status


def test_s4_ref_rejects():
    L = _ffi.lib()
    assert L.hx_s4_ref_fwd(4, 0, 4, 0.1, *([None] * 8), None) == _ffi.UnsupportedOperation.status
    assert L.hx_s4_ref_fwd(4, 16, 4, 0.1, *([None] * 8), None) == _ffi.InvalidInput.status
    assert L.hx_s4_ref_fwd(0, 16, 4, 0.1, *([None] * 8), None) == 0


def test_linear_rejects_bad_act():
    assert _ffi.lib().hx_linear_f32(2, 2, 2, None, None, None, 5, None, None) == _ffi.InvalidInput.status


def test_set_scan_variant_validation():
    assert _ffi.lib().hx_set_scan_variant(3) == _ffi.InvalidInput.status
    assert _ffi.lib().hx_set_scan_variant(0) == 0


def test_error_mapping_covers_tensor_error_variants():
    # status codes mirror tensor_core::TensorError (crates/tensor-core/src/error.rs:7-37)
    assert {c.__name__ for c in _ffi._BY_STATUS.values()} == {
        "ShapeMismatch", "InvalidDimension", "DeviceMismatch", "DTypeMismatch",
        "UnsupportedOperation", "AllocationFailed", "BackendError", "SerializationError",
        "InvalidInput", "InvalidCheckpoint"}
