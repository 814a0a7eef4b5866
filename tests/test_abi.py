"""The C-ABI library loads, exports every symbol include/helix_hip.h declares, and rejects bad
arguments on the host with the reference's TensorError variants — no GPU needed."""
import ctypes
import re
from pathlib import Path

import numpy as np
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
    assert L.hx_s4_ref_fwd(4, 0, 4, 0.1, *([None] * 7), None, 0, None) == _ffi.UnsupportedOperation.status
    assert L.hx_s4_ref_fwd(4, 16, 4, 0.1, *([None] * 7), None, 0, None) == _ffi.InvalidInput.status
    assert L.hx_s4_ref_fwd(0, 16, 4, 0.1, *([None] * 7), None, 0, None) == 0


def test_s4_discretize_is_the_reference_libm_formula():
    """hx_s4_discretize (host) = expf(f32(a_real*dt)) * cosf(f32(a_imag*dt)) in f32, as
    S4Block::discretize (crates/nn/src/ssm.rs:113-120) computes it; the oracle's restatement of
    the same function is pinned by the S4 reference-mode tests."""
    rng = np.random.default_rng(5)
    ar = rng.standard_normal(16).astype(np.float32)
    ai = rng.standard_normal(16).astype(np.float32) * np.float32(3)
    a = np.empty(16, np.float32)
    assert _ffi.lib().hx_s4_discretize(16, 0.1, ar.ctypes.data, ai.ctypes.data, a.ctypes.data) == 0
    tr = (ar * np.float32(0.1)).astype(np.float32)
    ti = (ai * np.float32(0.1)).astype(np.float32)
    ref = (np.exp(tr.astype(np.float64)) * np.cos(ti.astype(np.float64)))
    assert np.abs(a - ref).max() <= 2e-7 * np.abs(ref).max()
    # A_real = 0 (the reference's default init, ssm.rs:42): a = cos(dt * A_imag) exactly as f32 cosf
    ar0 = np.zeros(16, np.float32)
    assert _ffi.lib().hx_s4_discretize(16, 0.1, ar0.ctypes.data, ai.ctypes.data, a.ctypes.data) == 0
    assert np.abs(a - np.cos(ti.astype(np.float64))).max() <= 1.2e-7
    assert _ffi.lib().hx_s4_discretize(65, 0.1, None, None, None) == _ffi.UnsupportedOperation.status
    assert _ffi.lib().hx_s4_discretize(4, 0.1, None, None, None) == _ffi.InvalidInput.status


def test_workspace_sizes():
    L = _ffi.lib()
    # config 4 scan (batch 1, L 65536, d 2048): segmented, 16 segments x 3 x 32768 floats (end
    # states, entry states, decays)
    assert L.hx_selective_scan_workspace_size(1, 65536, 2048, 16, 0) == 16 * 3 * 2048 * 16 * 4
    # config 2 (batch 8, L 2048, d 1536) fills the GPU unsegmented: no workspace
    assert L.hx_selective_scan_workspace_size(8, 2048, 1536, 16, 0) == 0
    assert L.hx_selective_scan_workspace_size(1, 8192, 64, 7, 0) == 0  # generic kernel
    assert L.hx_s4_ref_workspace_size(64, 16, 100) >= (16 * 64 + 100 * 16) * 4
    assert L.hx_s4_ref_parallel_workspace_size(2048, 16, 65536) >= (2048 + 65536) * 16 * 4
    assert L.hx_s4d_workspace_size(1, 65536, 2048, 16) > 0
    assert L.hx_s4d_workspace_size(1, 100, 64, 8) == 0


def test_scan_ws_rejects_short_workspace():
    buf = (ctypes.c_uint8 * 64)()
    rc = _ffi.lib().hx_selective_scan_fwd_ws(1, 4, 4, 16, 0, 1, *([None] * 11), None, 64, None)
    assert rc == _ffi.InvalidInput.status  # NULL workspace with a size
    del buf


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
