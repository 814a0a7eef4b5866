"""ctypes binding of libhelix_hip.so — the Python twin of the Rust ``extern "C"`` block.

Every entry point declared in ``include/helix_hip.h`` is bound here with its exact C
signature. A non-zero status becomes the ``TensorError`` subclass matching the reference's
``tensor_core::TensorError`` variant (crates/tensor-core/src/error.rs:7-37), carrying the
library's ``hx_last_error()`` text. Nothing here computes: a missing library raises at import
time of the first call, there is no fallback path.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "libhelix_hip.so"


# ------------------------------------------------------------------ errors (TensorError mirror)
class TensorError(RuntimeError):
    """Base of the reference's TensorError enum (error.rs:7)."""
    status = -1


class ShapeMismatch(TensorError):
    status = 1


class InvalidDimension(TensorError):
    status = 2


class DeviceMismatch(TensorError):
    status = 3


class DTypeMismatch(TensorError):
    status = 4


class UnsupportedOperation(TensorError):
    status = 5


class AllocationFailed(TensorError):
    status = 6


class BackendError(TensorError):
    status = 7


class SerializationError(TensorError):
    status = 8


class InvalidInput(TensorError):
    status = 9


class InvalidCheckpoint(TensorError):
    status = 10


_BY_STATUS = {c.status: c for c in (ShapeMismatch, InvalidDimension, DeviceMismatch, DTypeMismatch,
                                    UnsupportedOperation, AllocationFailed, BackendError,
                                    SerializationError, InvalidInput, InvalidCheckpoint)}

HX_F32 = 0
HX_BF16 = 1

_i64 = ctypes.c_int64
_int = ctypes.c_int
_f = ctypes.c_float
_p = ctypes.c_void_p
_sz = ctypes.c_size_t

# name -> argtypes; every function returns int status except hx_last_error / hx_version.
SIGNATURES = {
    "hx_version": [],
    "hx_init": [_int],
    "hx_malloc": [ctypes.POINTER(ctypes.c_void_p), _sz],
    "hx_free": [_p],
    "hx_memcpy_h2d": [_p, _p, _sz],
    "hx_memcpy_d2h": [_p, _p, _sz],
    "hx_memcpy_d2d": [_p, _p, _sz, _p],
    "hx_sync": [],
    "hx_device_info": [_int, ctypes.POINTER(_int), ctypes.POINTER(_sz)],
    "hx_device_utilization": [_int, ctypes.POINTER(ctypes.c_double)],
    "hx_last_error": [],
    "hx_selective_scan_fwd": [_i64, _i64, _i64, _i64, _int, _int] + [_p] * 11 + [_p],
    "hx_selective_scan_workspace_size": [_i64, _i64, _i64, _i64, _int],
    "hx_selective_scan_fwd_ws": [_i64, _i64, _i64, _i64, _int, _int] + [_p] * 11 + [_p, _sz, _p],
    "hx_selective_scan_fwd_noalloc": [_i64, _i64, _i64, _i64, _int, _int] + [_p] * 11 + [_p],
    "hx_selective_state_update": [_i64, _i64, _i64, _int, _int] + [_p] * 10 + [_p],
    "hx_s4_discretize": [_i64, _f, _p, _p, _p],
    "hx_s4_ref_workspace_size": [_i64, _i64, _i64],
    "hx_s4_ref_fwd": [_i64, _i64, _i64, _f] + [_p] * 7 + [_p, _sz, _p],
    "hx_s4_ref_parallel_workspace_size": [_i64, _i64, _i64],
    "hx_s4_ref_fwd_parallel": [_i64, _i64, _i64, _f] + [_p] * 7 + [_p, _sz, _p],
    "hx_s4d_workspace_size": [_i64, _i64, _i64, _i64],
    "hx_s4d_complex_fwd": [_i64, _i64, _i64, _i64] + [_p] * 10 + [_p, _sz, _p],
    "hx_linear_f32": [_i64, _i64, _i64, _p, _p, _p, _int, _p, _p],
    "hx_matmul_f32": [_i64, _i64, _i64, _p, _p, _p, _p],
    "hx_gemm_bf16": [_i64, _i64, _i64, _p, _i64, _p, _i64, _p, _int, _int,
                     _p, _i64, _i64, _p, _i64, _i64, _p, _i64, _p],
    "hx_gemm_bf16_splitk": [_i64, _i64, _i64, _p, _i64, _p, _i64, _p, _int, _int,
                            _p, _i64, _i64, _p, _i64, _i64, _p, _i64, _int, _p, _sz, _p],
    "hx_conv1d_silu": [_i64, _i64, _i64, _i64, _int, _p, _i64, _p, _p, _p, _p],
    "hx_selective_scan_dtproj_fwd": [_i64, _i64, _i64, _i64] + [_p] * 12,
    "hx_mamba_block_workspace_size": [_i64, _i64, _i64, _i64, _i64],
    "hx_mamba_block_fwd": [_i64] * 7 + [_p] * 12 + [_sz, _p],
    "hx_embedding_fwd": [_i64, _i64, _i64, _p, _p, _p, _p],
    "hx_rmsnorm_fwd": [_i64, _i64, _p, _p, _f, _int, _p, _p],
    "hx_conv1d_step": [_i64, _i64, _i64, _int, _p, _i64, _p, _p, _p, _p, _p],
    "hx_mamba_layer_workspace_size": [_i64] * 6,
    "hx_mamba_layer_fwd": [_i64] * 7 + [_p, _p, _f] + [_p] * 11 + [_p, _sz, _p],
    "hx_mamba_layer_decode": [_i64] * 6 + [_p, _p, _f] + [_p] * 11 + [_p, _sz, _p],
    "hx_binary_f32": [_int, _i64, _p, _p, _p, _p],
    "hx_unary_f32": [_int, _i64, _p, _f, _p, _p],
    "hx_mean_axis_f32": [_i64, _i64, _i64, _int, _p, _p, _p],
    "hx_copy_strided_f32": [_int, _p, _p, _p, _p, _p, _p],
    "hx_fill_f32": [_i64, _f, _p, _p],
    "hx_eye_f32": [_i64, _p, _p],
    "hx_set_scan_variant": [_int],
    "hx_set_scan_segments": [_int],
    "hx_set_gemm_kernel": [_int],
    "hx_set_s4d_path": [_int],
    "hx_set_s4d_segments": [_int],
}

_lib = None


def lib() -> ctypes.CDLL:
    """Loads libhelix_hip.so (built by helixml_amd/build.py); raises if it is absent."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ImportError(
                f"{LIB_PATH} is not built; run `python -c 'import __graft_entry__ as g; g.build()'`")
        L = ctypes.CDLL(str(LIB_PATH))
        for name, args in SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = (ctypes.c_char_p if name == "hx_last_error" else
                          _sz if name.endswith("_workspace_size") else _int)
        _lib = L
    return _lib


def last_error() -> str:
    return lib().hx_last_error().decode(errors="replace")


def check(status: int, what: str = "") -> None:
    """Raises the TensorError variant for a non-zero hx status."""
    if status != 0:
        cls = _BY_STATUS.get(status, BackendError)
        raise cls(f"{what}: {last_error()}" if what else last_error())


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args), name)
