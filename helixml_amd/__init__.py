"""helixml_amd — MI355X (gfx950) backend for HelixML's SSM forward path.

The product is ``libhelix_hip.so`` (HIP kernels behind the C ABI in ``include/helix_hip.h``).
This package builds it (``build.py``), binds it (``_ffi.py``) and mirrors the reference's host
API over it: ``ssm`` holds the fused-op trait methods, ``nn`` the S4Block / MambaBlock /
Linear / RMSNorm modules with the reference's constructors and forward semantics.
"""
from ._ffi import (AllocationFailed, BackendError, DeviceMismatch, DTypeMismatch, InvalidDimension,
                   InvalidInput, ShapeMismatch, TensorError, UnsupportedOperation)

__all__ = [
    "TensorError", "ShapeMismatch", "InvalidDimension", "DeviceMismatch", "DTypeMismatch",
    "UnsupportedOperation", "AllocationFailed", "BackendError", "InvalidInput",
]
