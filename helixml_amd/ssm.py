"""Functional host layer over the C ABI — the ``TensorSsm`` extension-trait methods.

The reference composes its SSM blocks from generic tensor-trait calls
(crates/tensor-core/src/tensor.rs:7-275). Fusing them needs one extension trait whose methods
the HIP backend overrides; these functions are those methods for torch device tensors (torch
supplies device memory and the stream only; every value is computed by libhelix_hip.so).

Shape and dtype checks run here first and raise the reference's ``TensorError`` variants
(``ShapeMismatch``, ``DTypeMismatch`` …) before anything reaches the device, mirroring how
CpuTensor validates before computing (backend-cpu/src/lib.rs:570-576, 648-656).
"""
from __future__ import annotations

from typing import Optional

import torch

from . import _ffi
from ._ffi import DTypeMismatch, InvalidInput, ShapeMismatch

_STORAGE = {torch.float32: _ffi.HX_F32, torch.bfloat16: _ffi.HX_BF16}


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else t.data_ptr()


def _stream(stream) -> int:
    if stream is None:
        return torch.cuda.current_stream().cuda_stream
    return stream.cuda_stream if hasattr(stream, "cuda_stream") else int(stream)


def _need(t: Optional[torch.Tensor], name: str, shape, dtype) -> None:
    if t is None:
        return
    if not t.is_cuda:
        raise InvalidInput(f"{name} must be a device tensor")
    if tuple(t.shape) != tuple(shape):
        raise ShapeMismatch(f"{name}: expected {list(shape)}, got {list(t.shape)}")
    if t.dtype != dtype:
        raise DTypeMismatch(f"{name}: expected {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise InvalidInput(f"{name} must be contiguous")


def selective_scan_fwd(u, delta, A, B, C, D=None, z=None, dt_bias=None, delta_softplus=True,
                       init_state=None, return_last_state=False, out=None, stream=None):
    """Fused selective scan (hx_selective_scan_fwd). u, delta, z: [batch, L, dim];
    B, C: [batch, L, dstate]; A: [dim, dstate] fp32; D, dt_bias: [dim] fp32."""
    if u.dim() != 3:
        raise ShapeMismatch(f"u: expected 3 dims [batch, seqlen, dim], got {list(u.shape)}")
    bt, L, dim = u.shape
    if A.dim() != 2:
        raise ShapeMismatch(f"A: expected [dim, dstate], got {list(A.shape)}")
    N = A.shape[1]
    if u.dtype not in _STORAGE:
        raise DTypeMismatch(f"u: storage dtype {u.dtype} is neither float32 nor bfloat16")
    st = u.dtype
    _need(u, "u", (bt, L, dim), st)
    _need(delta, "delta", (bt, L, dim), st)
    _need(A, "A", (dim, N), torch.float32)
    _need(B, "B", (bt, L, N), st)
    _need(C, "C", (bt, L, N), st)
    _need(D, "D", (dim,), torch.float32)
    _need(z, "z", (bt, L, dim), st)
    _need(dt_bias, "dt_bias", (dim,), torch.float32)
    _need(init_state, "init_state", (bt, dim, N), torch.float32)
    if out is None:
        out = torch.empty_like(u)
    _need(out, "out", (bt, L, dim), st)
    last = torch.empty((bt, dim, N), device=u.device, dtype=torch.float32) if return_last_state else None
    _ffi.call("hx_selective_scan_fwd", bt, L, dim, N, _STORAGE[st], int(bool(delta_softplus)),
              _ptr(u), _ptr(delta), _ptr(A), _ptr(B), _ptr(C), _ptr(D), _ptr(z), _ptr(dt_bias),
              _ptr(out), _ptr(init_state), _ptr(last), _stream(stream))
    return (out, last) if return_last_state else out


def selective_state_update(state, u, delta, A, B, C, D=None, z=None, dt_bias=None,
                           delta_softplus=True, out=None, stream=None):
    """One decode step (hx_selective_state_update); updates ``state`` [batch, dim, dstate] in place.
    u, delta, z, out: [batch, dim]; B, C: [batch, dstate]."""
    bt, dim = u.shape
    N = A.shape[1]
    st = u.dtype
    if st not in _STORAGE:
        raise DTypeMismatch(f"u: storage dtype {st} is neither float32 nor bfloat16")
    _need(state, "state", (bt, dim, N), torch.float32)
    _need(delta, "delta", (bt, dim), st)
    _need(A, "A", (dim, N), torch.float32)
    _need(B, "B", (bt, N), st)
    _need(C, "C", (bt, N), st)
    _need(D, "D", (dim,), torch.float32)
    _need(z, "z", (bt, dim), st)
    _need(dt_bias, "dt_bias", (dim,), torch.float32)
    if out is None:
        out = torch.empty_like(u)
    _ffi.call("hx_selective_state_update", bt, dim, N, _STORAGE[st], int(bool(delta_softplus)),
              _ptr(state), _ptr(u), _ptr(delta), _ptr(A), _ptr(B), _ptr(C), _ptr(D), _ptr(z),
              _ptr(dt_bias), _ptr(out), _stream(stream))
    return out


def s4_ref_fwd(x, a_real, a_imag, B, C, D, gate=None, dt=0.1, stream=None):
    """Reference-mode S4Block::forward_ssm (crates/nn/src/ssm.rs:138-186) on x [d_model, L];
    returns y with memory [L, d_model] (the reference's shape field is [d_model, L])."""
    M, L = x.shape
    N = a_real.shape[0]
    f = torch.float32
    _need(x, "x", (M, L), f)
    _need(a_real, "A_real", (N,), f)
    _need(a_imag, "A_imag", (N,), f)
    _need(B, "B", (N, M), f)
    _need(C, "C", (M, N), f)
    _need(D, "D", (M,), f)
    _need(gate, "gate", (M,), f)
    y = torch.empty((L, M), device=x.device, dtype=f)
    _ffi.call("hx_s4_ref_fwd", M, N, L, float(dt), _ptr(x), _ptr(a_real), _ptr(a_imag), _ptr(B),
              _ptr(C), _ptr(D), _ptr(gate), _ptr(y), _stream(stream))
    return y


def s4d_complex_fwd(x, dt, a_re, a_im, B_re, B_im, C_re, C_im, D=None, stream=None):
    """S4D diagonal complex recurrence (hx_s4d_complex_fwd); x, y: [batch, L, dim]."""
    bt, L, dim = x.shape
    N = a_re.shape[1]
    f = torch.float32
    _need(x, "x", (bt, L, dim), f)
    _need(dt, "dt", (dim,), f)
    for name, t in (("a_re", a_re), ("a_im", a_im), ("B_re", B_re), ("B_im", B_im),
                    ("C_re", C_re), ("C_im", C_im)):
        _need(t, name, (dim, N), f)
    _need(D, "D", (dim,), f)
    y = torch.empty_like(x)
    _ffi.call("hx_s4d_complex_fwd", bt, L, dim, N, _ptr(x), _ptr(dt), _ptr(a_re), _ptr(a_im),
              _ptr(B_re), _ptr(B_im), _ptr(C_re), _ptr(C_im), _ptr(D), _ptr(y), _stream(stream))
    return y


def linear(X, W, bias=None, act=0, stream=None):
    """nn::Linear::forward (crates/nn/src/lib.rs:120-134); W is [out, in]."""
    R, IN = X.shape
    OUT = W.shape[0]
    if W.shape[1] != IN:
        # CpuTensor::matmul's mismatch error: expected [a_cols], actual [b_rows] (lib.rs:651-656)
        raise ShapeMismatch(f"expected {[IN]}, got {[W.shape[1]]}")
    f = torch.float32
    _need(X, "X", (R, IN), f)
    _need(W, "W", (OUT, IN), f)
    _need(bias, "bias", (OUT,), f)
    Y = torch.empty((R, OUT), device=X.device, dtype=f)
    _ffi.call("hx_linear_f32", R, IN, OUT, _ptr(X), _ptr(W), _ptr(bias), int(act), _ptr(Y),
              _stream(stream))
    return Y


def matmul(A, B, stream=None):
    """CpuTensor::matmul 2-D x 2-D (crates/backend-cpu/src/lib.rs:644-678)."""
    M, K = A.shape
    K2, N = B.shape
    if K != K2:
        raise ShapeMismatch(f"expected {[K]}, got {[K2]}")
    f = torch.float32
    _need(A, "A", (M, K), f)
    _need(B, "B", (K, N), f)
    Y = torch.empty((M, N), device=A.device, dtype=f)
    _ffi.call("hx_matmul_f32", M, K, N, _ptr(A), _ptr(B), _ptr(Y), _stream(stream))
    return Y


def gemm_bf16(X, W, bias=None, act=0, out_dtype=torch.bfloat16, splits=None, stream=None):
    """Matrix-core GEMM Y = X . W^T (+ bias)(, SiLU) (hx_gemm_bf16). X [M, K], W [N, K] bf16
    (row-major; X may be a row-strided view). splits=(s1[, s2]) returns the column blocks
    [0, s1), [s1, s2), [s2, N) as separate contiguous tensors."""
    M, K = X.shape
    N = W.shape[0]
    if W.shape[1] != K:
        raise ShapeMismatch(f"expected {[K]}, got {[W.shape[1]]}")
    if X.dtype != torch.bfloat16 or W.dtype != torch.bfloat16:
        raise DTypeMismatch("gemm_bf16: X and W must be bfloat16")
    if X.stride(1) != 1 or W.stride(1) != 1:
        raise InvalidInput("gemm_bf16: X and W need unit column stride")
    _need(bias, "bias", (N,), torch.float32)
    cuts = [0] + list(splits or []) + [N]
    outs = [torch.empty((M, cuts[i + 1] - cuts[i]), device=X.device, dtype=out_dtype)
            for i in range(len(cuts) - 1)]
    ys = outs + [None] * (3 - len(outs))
    s1 = cuts[1] if len(cuts) > 2 else N
    s2 = cuts[2] if len(cuts) > 3 else N
    od = _STORAGE[out_dtype]
    _ffi.call("hx_gemm_bf16", M, N, K, _ptr(X), X.stride(0), _ptr(W), W.stride(0), _ptr(bias),
              int(act), od, _ptr(ys[0]), ys[0].shape[1], s1,
              _ptr(ys[1]), ys[1].shape[1] if ys[1] is not None else 0, s2,
              _ptr(ys[2]), ys[2].shape[1] if ys[2] is not None else 0, _stream(stream))
    return outs[0] if len(outs) == 1 else tuple(outs)


def set_scan_variant(v: int) -> None:
    _ffi.call("hx_set_scan_variant", int(v))


def set_scan_segments(n: int) -> None:
    _ffi.call("hx_set_scan_segments", int(n))
