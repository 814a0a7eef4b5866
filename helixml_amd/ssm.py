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

import functools
from typing import Optional

import numpy as np

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


def _torch_stream(stream):
    """The torch stream a launch goes to: the current stream for None, a torch stream as given,
    anything else (a raw hipStream_t handle) wrapped as an external stream."""
    if stream is None:
        return torch.cuda.current_stream()
    if isinstance(stream, torch.cuda.Stream):
        return stream
    return torch.cuda.ExternalStream(int(getattr(stream, "cuda_stream", stream)))


def on_launch_stream(fn):
    """Runs a wrapper with its launch stream current, so every temporary it allocates (outputs,
    workspaces) belongs to the stream its kernels run on: torch's caching allocator then cannot
    hand that memory to another allocation while those kernels may still use it."""
    @functools.wraps(fn)
    def run(*args, stream=None, **kwargs):
        ts = _torch_stream(stream)
        with torch.cuda.stream(ts):
            return fn(*args, stream=ts, **kwargs)
    run.on_launch_stream = True
    return run


def keep_for_stream(t: Optional[torch.Tensor], stream) -> None:
    """Marks a persistent buffer (a workspace kept between calls) as used on ``stream``, so that
    replacing it later cannot recycle its memory while work queued there still reads it."""
    if t is not None and not torch.cuda.is_current_stream_capturing():
        t.record_stream(stream)


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


def selective_scan_workspace_size(batch, seqlen, dim, dstate, dtype=torch.float32):
    """Bytes of scratch hx_selective_scan_fwd_ws needs (0 when the sequence is not segmented)."""
    return int(_ffi.lib().hx_selective_scan_workspace_size(batch, seqlen, dim, dstate, _STORAGE[dtype]))


@on_launch_stream
def selective_scan_fwd(u, delta, A, B, C, D=None, z=None, dt_bias=None, delta_softplus=True,
                       init_state=None, return_last_state=False, out=None, workspace=None,
                       stream=None):
    """Fused selective scan (hx_selective_scan_fwd_ws). u, delta, z: [batch, L, dim];
    B, C: [batch, L, dstate]; A: [dim, dstate] fp32; D, dt_bias: [dim] fp32. ``workspace``: a
    uint8 device tensor of at least selective_scan_workspace_size(...) bytes for the segmented
    long-sequence path; allocated here (by torch, outside the library) when not given."""
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
    need = selective_scan_workspace_size(bt, L, dim, N, st)
    if need and (workspace is None or workspace.numel() < need):
        workspace = torch.empty(need, device=u.device, dtype=torch.uint8)
    nbytes = workspace.numel() if (need and workspace is not None) else 0
    _ffi.call("hx_selective_scan_fwd_ws", bt, L, dim, N, _STORAGE[st], int(bool(delta_softplus)),
              _ptr(u), _ptr(delta), _ptr(A), _ptr(B), _ptr(C), _ptr(D), _ptr(z), _ptr(dt_bias),
              _ptr(out), _ptr(init_state), _ptr(last), _ptr(workspace) if nbytes else None, nbytes,
              _stream(stream))
    return (out, last) if return_last_state else out


@on_launch_stream
def selective_scan_dtproj_fwd(u, dt_lo, w_dt, A, B, C, D, z, dt_bias, return_last_state=False,
                              out=None, stream=None):
    """The block's dt projection and selective scan in one launch (hx_selective_scan_dtproj_fwd):
    dt = bf16(dt_lo . w_dt^T) formed per 16-step chunk on the matrix core, then the scan with
    softplus(dt + dt_bias) and the SiLU(z) gate from a zero state. bf16 u, z, out [batch, L, dim],
    dt_lo [batch, L, dt_rank], w_dt [dim, dt_rank], B, C [batch, L, 16]; A [dim, 16], D, dt_bias
    [dim] fp32."""
    bt, L, dim = u.shape
    r = dt_lo.shape[-1]
    bf = torch.bfloat16
    _need(u, "u", (bt, L, dim), bf)
    _need(dt_lo, "dt_lo", (bt, L, r), bf)
    _need(w_dt, "w_dt", (dim, r), bf)
    _need(A, "A", (dim, 16), torch.float32)
    _need(B, "B", (bt, L, 16), bf)
    _need(C, "C", (bt, L, 16), bf)
    _need(D, "D", (dim,), torch.float32)
    _need(z, "z", (bt, L, dim), bf)
    _need(dt_bias, "dt_bias", (dim,), torch.float32)
    if out is None:
        out = torch.empty_like(u)
    _need(out, "out", (bt, L, dim), bf)
    last = torch.empty((bt, dim, 16), device=u.device, dtype=torch.float32) if return_last_state else None
    _ffi.call("hx_selective_scan_dtproj_fwd", bt, L, dim, r, _ptr(u), _ptr(dt_lo), _ptr(w_dt), _ptr(A),
              _ptr(B), _ptr(C), _ptr(D), _ptr(z), _ptr(dt_bias), _ptr(out), _ptr(last), _stream(stream))
    return (out, last) if return_last_state else out


@on_launch_stream
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


def s4_discretize(a_real, a_imag, dt=0.1, device=None):
    """S4Block::discretize's decay (crates/nn/src/ssm.rs:113-120) through hx_s4_discretize:
    a = expf(a_real*dt) * cosf(a_imag*dt) computed on the host with the reference's libm, returned
    as a float32 device tensor. Reads a_real/a_imag back if they live on the device (one copy);
    callers that run many forwards with the same parameters compute it once."""
    ar = np.ascontiguousarray(a_real.detach().float().cpu().numpy())
    ai = np.ascontiguousarray(a_imag.detach().float().cpu().numpy())
    n = ar.shape[0]
    a = np.empty(n, np.float32)
    _ffi.call("hx_s4_discretize", n, float(dt), ar.ctypes.data, ai.ctypes.data, a.ctypes.data)
    return torch.from_numpy(a).to(device if device is not None else a_real.device)


@on_launch_stream
def s4_ref_fwd(x, a_real, a_imag, B, C, D, gate=None, dt=0.1, parallel=False, a=None,
               workspace=None, stream=None):
    """Reference-mode S4Block::forward_ssm (crates/nn/src/ssm.rs:138-186) on x [d_model, L];
    returns y with memory [L, d_model] (the reference's shape field is [d_model, L]).
    parallel=False: bit-identical to CpuTensor (hx_s4_ref_fwd); parallel=True: time-parallel
    chunked recurrence for long L, equal to rounding (hx_s4_ref_fwd_parallel, dstate <= 16).
    ``a``: the discretised decay (s4_discretize(a_real, a_imag, dt)); computed here when None."""
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
    if a is None:
        a = s4_discretize(a_real, a_imag, dt, device=x.device)
    _need(a, "a", (N,), f)
    y = torch.empty((L, M), device=x.device, dtype=f)
    size_fn = "hx_s4_ref_parallel_workspace_size" if parallel else "hx_s4_ref_workspace_size"
    need = int(getattr(_ffi.lib(), size_fn)(M, N, L))
    if workspace is None or workspace.numel() < need:
        workspace = torch.empty(max(need, 1), device=x.device, dtype=torch.uint8)
    _ffi.call("hx_s4_ref_fwd_parallel" if parallel else "hx_s4_ref_fwd", M, N, L, float(dt), _ptr(x),
              _ptr(a), _ptr(B), _ptr(C), _ptr(D), _ptr(gate), _ptr(y), _ptr(workspace),
              workspace.numel(), _stream(stream))
    return y


@on_launch_stream
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
    need = int(_ffi.lib().hx_s4d_workspace_size(bt, L, dim, N))
    ws = torch.empty(need, device=x.device, dtype=torch.uint8) if need else None
    _ffi.call("hx_s4d_complex_fwd", bt, L, dim, N, _ptr(x), _ptr(dt), _ptr(a_re), _ptr(a_im),
              _ptr(B_re), _ptr(B_im), _ptr(C_re), _ptr(C_im), _ptr(D), _ptr(y), _ptr(ws), need,
              _stream(stream))
    return y


@on_launch_stream
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


@on_launch_stream
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


@on_launch_stream
def gemm_bf16(X, W, bias=None, act=0, out_dtype=torch.bfloat16, splits=None, stream=None,
              k_splits=None):
    """Matrix-core GEMM Y = X . W^T (+ bias)(, SiLU) (hx_gemm_bf16). X [M, K], W [N, K] bf16
    (row-major; X may be a row-strided view). splits=(s1[, s2]) returns the column blocks
    [0, s1), [s1, s2), [s2, N) as separate contiguous tensors. k_splits=S runs the split-K form
    (hx_gemm_bf16_splitk) with an fp32 workspace of S * M * N floats."""
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
    args = (M, N, K, _ptr(X), X.stride(0), _ptr(W), W.stride(0), _ptr(bias), int(act), od,
            _ptr(ys[0]), ys[0].shape[1], s1, _ptr(ys[1]), ys[1].shape[1] if ys[1] is not None else 0,
            s2, _ptr(ys[2]), ys[2].shape[1] if ys[2] is not None else 0)
    if k_splits:
        ws = torch.empty(int(k_splits) * M * N, device=X.device, dtype=torch.float32)
        _ffi.call("hx_gemm_bf16_splitk", *args, int(k_splits), _ptr(ws), ws.numel() * 4, _stream(stream))
    else:
        _ffi.call("hx_gemm_bf16", *args, _stream(stream))
    return outs[0] if len(outs) == 1 else tuple(outs)


def set_scan_variant(v: int) -> None:
    _ffi.call("hx_set_scan_variant", int(v))


def set_scan_segments(n: int) -> None:
    _ffi.call("hx_set_scan_segments", int(n))


def set_gemm_kernel(k: int) -> None:
    _ffi.call("hx_set_gemm_kernel", int(k))


def set_s4d_path(path: int) -> None:
    _ffi.call("hx_set_s4d_path", int(path))


def set_s4d_segments(n: int) -> None:
    _ffi.call("hx_set_s4d_segments", int(n))


@on_launch_stream
def conv1d_silu(x, weight, bias=None, out=None, stream=None):
    """Causal depthwise conv1d + bias + SiLU (hx_conv1d_silu). x [batch, L, dim] (rows may be
    strided, e.g. the x half of in_proj's output), weight [dim, width] fp32, bias [dim] fp32."""
    bt, L, dim = x.shape
    if x.dtype not in _STORAGE:
        raise DTypeMismatch(f"x: storage dtype {x.dtype} is neither float32 nor bfloat16")
    if x.stride(2) != 1 or x.stride(0) != L * x.stride(1):
        raise InvalidInput("conv1d_silu: x needs unit channel stride and uniform row stride")
    _need(weight, "weight", (dim, weight.shape[1]), torch.float32)
    _need(bias, "bias", (dim,), torch.float32)
    if out is None:
        out = torch.empty((bt, L, dim), device=x.device, dtype=x.dtype)
    _need(out, "out", (bt, L, dim), x.dtype)
    _ffi.call("hx_conv1d_silu", bt, L, dim, weight.shape[1], _STORAGE[x.dtype], _ptr(x),
              x.stride(1), _ptr(weight), _ptr(bias), _ptr(out), _stream(stream))
    return out


def mamba_block_workspace_size(batch, seqlen, d_inner, dt_rank, dstate) -> int:
    return int(_ffi.lib().hx_mamba_block_workspace_size(batch, seqlen, d_inner, dt_rank, dstate))


@on_launch_stream
def mamba_block_fwd(x, w_in, conv_w, conv_b, w_x, w_dt, dt_bias, A, D, w_out, workspace=None,
                    out=None, stream=None):
    """Full Mamba block forward (hx_mamba_block_fwd), bf16 storage. x [batch, L, d_model];
    w_in [2*d_inner, d_model], w_x [dt_rank + 2*dstate, d_inner], w_dt [d_inner, dt_rank],
    w_out [d_model, d_inner] bf16; conv_w [d_inner, d_conv], conv_b, dt_bias, D [d_inner],
    A [d_inner, dstate] fp32. ``workspace``: a uint8 device tensor of at least
    mamba_block_workspace_size(...) bytes (allocated here if None)."""
    bt, L, dm = x.shape
    di, dt_rank = w_dt.shape
    N = A.shape[1]
    bf = torch.bfloat16
    _need(x, "x", (bt, L, dm), bf)
    _need(w_in, "w_in", (2 * di, dm), bf)
    _need(conv_w, "conv_w", (di, conv_w.shape[1]), torch.float32)
    _need(conv_b, "conv_b", (di,), torch.float32)
    _need(w_x, "w_x", (dt_rank + 2 * N, di), bf)
    _need(w_dt, "w_dt", (di, dt_rank), bf)
    _need(dt_bias, "dt_bias", (di,), torch.float32)
    _need(A, "A", (di, N), torch.float32)
    _need(D, "D", (di,), torch.float32)
    _need(w_out, "w_out", (dm, di), bf)
    ws_bytes = mamba_block_workspace_size(bt, L, di, dt_rank, N)
    if workspace is None:
        workspace = torch.empty(ws_bytes, device=x.device, dtype=torch.uint8)
    if out is None:
        out = torch.empty((bt, L, dm), device=x.device, dtype=bf)
    _need(out, "out", (bt, L, dm), bf)
    _ffi.call("hx_mamba_block_fwd", bt, L, dm, di, N, dt_rank, conv_w.shape[1], _ptr(x), _ptr(w_in),
              _ptr(conv_w), _ptr(conv_b), _ptr(w_x), _ptr(w_dt), _ptr(dt_bias), _ptr(A), _ptr(D),
              _ptr(w_out), _ptr(out), _ptr(workspace), workspace.numel() * workspace.element_size(),
              _stream(stream))
    return out


class MambaBlock:
    """Device-resident Mamba block with the reference constructor's arguments
    (``MambaBlock::new(d_model, d_state, d_conv, expand)``, crates/nn/src/lib.rs:847) and the
    parameters that constructor names (A, D, delta/B/C projections, in ("gate") and out
    projections) laid out for the fused path: w_in = in_proj, w_x = x_proj (dt_lo | B | C rows),
    w_dt = dt_proj, dt_rank = ceil(d_model / 16). ``forward`` is hx_mamba_block_fwd; the
    workspace is kept between calls and regrown when a larger input arrives."""

    def __init__(self, d_model, d_state=16, d_conv=4, expand=2, dt_rank=None, device="cuda",
                 generator=None):
        self.d_model, self.d_state, self.d_conv, self.expand = d_model, d_state, d_conv, expand
        self.d_inner = d_model * expand
        self.dt_rank = dt_rank or -(-d_model // 16)
        di, r, N = self.d_inner, self.dt_rank, d_state
        g = generator
        f32, bf = torch.float32, torch.bfloat16

        def normal(shape, std):
            return (torch.randn(shape, generator=g) * std)

        self.w_in = normal((2 * di, d_model), (2.0 / d_model) ** 0.5).to(device, bf)
        self.conv_w = ((torch.rand((di, d_conv), generator=g) * 2 - 1) / d_conv ** 0.5).to(device, f32)
        self.conv_b = ((torch.rand(di, generator=g) * 2 - 1) / d_conv ** 0.5).to(device, f32)
        self.w_x = normal((r + 2 * N, di), (2.0 / di) ** 0.5).to(device, bf)
        self.w_dt = normal((di, r), r ** -0.5).to(device, bf)
        # dt = softplus(dt_proj + dt_bias) starts log-uniform in [1e-3, 1e-1]
        dt0 = torch.exp(torch.rand(di, generator=g) * (torch.log(torch.tensor(0.1)) -
                                                          torch.log(torch.tensor(1e-3)))
                        + torch.log(torch.tensor(1e-3)))
        self.dt_bias = (dt0 + torch.log(-torch.expm1(-dt0))).to(device, f32)
        self.A = (-torch.arange(1, N + 1, dtype=f32)).repeat(di, 1).to(device)
        self.D = torch.ones(di, dtype=f32).to(device)
        self.w_out = normal((d_model, di), (2.0 / di) ** 0.5).to(device, bf)
        self._ws = None

    def parameters(self):
        return dict(w_in=self.w_in, conv_w=self.conv_w, conv_b=self.conv_b, w_x=self.w_x,
                    w_dt=self.w_dt, dt_bias=self.dt_bias, A=self.A, D=self.D, w_out=self.w_out)

    @on_launch_stream
    def forward(self, x, out=None, stream=None):
        """Calls that share this block's workspace must be ordered on one stream (it holds
        intermediates only during a call)."""
        bt, L, _ = x.shape
        need = mamba_block_workspace_size(bt, L, self.d_inner, self.dt_rank, self.d_state)
        if self._ws is None or self._ws.numel() < need:
            self._ws = torch.empty(need, device=x.device, dtype=torch.uint8)
        keep_for_stream(self._ws, stream)
        return mamba_block_fwd(x, workspace=self._ws, out=out, stream=stream, **self.parameters())

    __call__ = forward
