"""CPU oracle for the SSM forward path — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
this package; the product library (``helixml_amd``, ``libhelix_hip.so``) never does.

``liboracle.so`` (built from ``hx_oracle.c`` / ``hx_oracle_omp.c`` by ``make -C oracle``) holds
the plain-C restatement of the reference's CPU arithmetic; this module wraps it for numpy.
``numpy_*`` functions are a second, independent float64 restatement used to cross-check the C
one (tests/test_oracle.py).

Pinning status of each function (how tests/test_oracle.py pins it):
  matmul, linear        reference KATs ones[2,3].ones[3,4] == 3 and ones+ones == 2
                        (backend-cpu/src/lib.rs:1733-1758), numpy float64
  silu                  closed form x*sigmoid(x), special values
  s4_ref_fwd(_f64)      zero input, impulse response, step response (geometric series),
                        linearity, B=0 -> D*u, a=1 -> prefix sum, numpy float64 brute force
  ssm_mamba_fwd         composition: matmul + s4_ref_fwd + gate (each pinned above)
  mamba_mlp             composition of linear/silu, numpy float64
  rmsnorm               closed form on constant rows, numpy float64
  selective_scan(_f64)  B=0/C=0 -> D*u*silu(z); A=0 -> prefix sum; N=1 constant inputs ->
                        geometric series; split-sequence == whole (state hand-off);
                        decode steps == prefill; f32 vs f64; numpy float64
  conv1d_silu           width 1 == silu(w*x+b); unit impulse -> time-reversed taps; causality
                        (future inputs change nothing); numpy float64 np.convolve per channel
  lm_prefill/decode     compositions of the pinned pieces above (embedding = array indexing);
                        cross-checked by decode-after-prefill == prefill of the longer sequence
  conv1d_step           one step == the last output of conv1d_silu over the window
  mamba_block           composition of linear + conv1d_silu + selective_scan (each pinned),
                        bf16 rounding at the storage points; cross-checked against
                        numpy_mamba_block (float64, same storage rounding)
  s4d_complex           impulse response 2*Re(sum C Abar^t Bbar), constant-input steady state
  unary                 special values (exp 0 = 1, cos 0 = 1, sin 0 = 0, log 1 = 0, sqrt of
                        squares), float64 within one f32 ulp, silu/sigmoid formulas
  mean_axis             constant and small-integer rows (exact); the summation order by a
                        crafted row whose sum is 6 in ndarray's eight-accumulator fold and 3 in
                        sequential order (hand-derived from the fold), and the same values as a
                        column (sequential order off the contiguous axis: 3)
  rmsnorm_ref           composition of unary/mean (pinned above); equals rmsnorm to rounding
  broadcast_to, stack,  numpy's broadcast_to / concatenate / stack / transpose / slicing on the
  transpose, slice2d,   cases the reference computes correctly; the generic broadcast's stride
  cat1d                 quirk on a hand-derived case (src [2, 3] -> [1, 1, 2, 3])
  r_s4_forward_ssm,     the reference's execution shape (allocation per op, copying slices,
  r_mamba_mlp           reshapes and stack, hx_oracle_ref.c) for the CPU-baseline timing;
                        bit-identical to s4_ref_fwd / mamba_mlp (checked in tests)
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

_lib = None

_f = ctypes.c_float
_i64 = ctypes.c_int64
_int = ctypes.c_int
_p = ctypes.c_void_p


def build() -> Path:
    """Compiles liboracle.so with the Makefile next to this file."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        sig = {
            "oracle_matmul": [_i64, _i64, _i64, _p, _p, _p],
            "oracle_silu": [_i64, _p, _p],
            "oracle_linear": [_i64, _i64, _i64, _p, _p, _p, _int, _p],
            "oracle_mamba_mlp": [_i64, _i64, _i64, _p, _p, _p, _p, _p, _p, _p],
            "oracle_rmsnorm": [_i64, _i64, _p, _p, _f, _p],
            "oracle_s4_ref_fwd": [_i64, _i64, _i64, _f, _p, _p, _p, _p, _p, _p, _p, _p, _p],
            "oracle_s4_ref_fwd_f64": [_i64, _i64, _i64, _f, _p, _p, _p, _p, _p, _p, _p, _p, _p],
            "oracle_ssm_mamba_fwd": [_i64, _i64, _f, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p],
            "oracle_selective_scan": [_i64, _i64, _i64, _i64, _int] + [_p] * 11,
            "oracle_selective_scan_f64": [_i64, _i64, _i64, _i64, _int] + [_p] * 11,
            "oracle_selective_state_update": [_i64, _i64, _i64, _int] + [_p] * 10,
            "oracle_s4d_complex": [_i64, _i64, _i64, _i64] + [_p] * 10,
            "oracle_selective_scan_omp": [_i64, _i64, _i64, _i64, _int] + [_p] * 11 + [_int],
            "oracle_selective_state_update_omp": [_i64, _i64, _i64, _int] + [_p] * 10 + [_int],
            "oracle_linear_omp": [_i64, _i64, _i64, _p, _p, _p, _int, _p, _p, _int],
            "oracle_conv1d_silu_omp": [_i64, _i64, _i64, _i64, _p, _i64, _p, _p, _p, _int],
            "oracle_rmsnorm_omp": [_i64, _i64, _p, _p, _f, _p, _int],
            "oracle_s4d_complex_omp": [_i64, _i64, _i64, _i64] + [_p] * 10 + [_int],
            "oracle_r_linear": [_i64, _i64, _i64, _p, _p, _p, _p],
            "oracle_s4_ref_fwd_omp": [_i64, _i64, _i64, _f] + [_p] * 10 + [_int],
            "oracle_max_threads": [],
            "oracle_conv1d_silu": [_i64, _i64, _i64, _i64, _p, _i64, _p, _p, _p],
            "oracle_r_s4_forward_ssm": [_i64, _i64, _i64, _f] + [_p] * 9,
            "oracle_r_mamba_mlp": [_i64, _i64, _i64] + [_p] * 6,
            "oracle_unary": [_int, _i64, _p, _f, _p],
            "oracle_mean_axis": [_i64, _i64, _i64, _int, _p, _p],
            "oracle_rmsnorm_ref": [_i64, _i64, _p, _p, _f, _p, _p],
        }
        for name, args in sig.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = _int if name == "oracle_max_threads" else None
        _lib = L
    return _lib


def _ptr(a):
    if a is None:
        return None
    return a.ctypes.data_as(ctypes.c_void_p)


def _f32(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.float32)


# ------------------------------------------------------------------ C restatement wrappers

def matmul(A, B):
    A, B = _f32(A), _f32(B)
    M, K = A.shape
    K2, N = B.shape
    assert K == K2
    Y = np.empty((M, N), np.float32)
    lib().oracle_matmul(M, K, N, _ptr(A), _ptr(B), _ptr(Y))
    return Y


def silu(x):
    x = _f32(x)
    y = np.empty_like(x)
    lib().oracle_silu(x.size, _ptr(x), _ptr(y))
    return y


def linear(X, W, bias=None, act=0):
    X, W, bias = _f32(X), _f32(W), _f32(bias)
    R, IN = X.shape
    OUT = W.shape[0]
    Y = np.empty((R, OUT), np.float32)
    lib().oracle_linear(R, IN, OUT, _ptr(X), _ptr(W), _ptr(bias), act, _ptr(Y))
    return Y


def mamba_mlp(X, Wg, bg, Wo, bo):
    X, Wg, bg, Wo, bo = map(_f32, (X, Wg, bg, Wo, bo))
    R, dm = X.shape
    di = Wg.shape[0]
    tmp = np.empty((R, di), np.float32)
    Y = np.empty((R, dm), np.float32)
    lib().oracle_mamba_mlp(R, dm, di, _ptr(X), _ptr(Wg), _ptr(bg), _ptr(Wo), _ptr(bo), _ptr(tmp), _ptr(Y))
    return Y


def rmsnorm(X, w, eps):
    X, w = _f32(X), _f32(w)
    R, Dm = X.shape
    Y = np.empty_like(X)
    lib().oracle_rmsnorm(R, Dm, _ptr(X), _ptr(w), eps, _ptr(Y))
    return Y


def s4_ref_fwd(x, a_real, a_imag, B, C, D, gate=None, dt=0.1, f64=False):
    """x [M, L] -> y memory [L, M] (see hx_oracle.c); f64=True: the double restatement."""
    x, a_real, a_imag, B, C, D, gate = map(_f32, (x, a_real, a_imag, B, C, D, gate))
    M, L = x.shape
    N = a_real.shape[0]
    dt_ = np.float64 if f64 else np.float32
    y = np.empty((L, M), dt_)
    work = np.empty(3 * N + M, dt_)
    fn = lib().oracle_s4_ref_fwd_f64 if f64 else lib().oracle_s4_ref_fwd
    fn(M, N, L, dt, _ptr(x), _ptr(a_real), _ptr(a_imag), _ptr(B), _ptr(C), _ptr(D), _ptr(gate),
       _ptr(y), _ptr(work))
    return y


def s4_ref_fwd_omp(x, a_real, a_imag, B, C, D, gate=None, dt=0.1, threads=0):
    """s4_ref_fwd's values bit for bit, with the projection and readout spread over threads
    (hx_oracle_omp.c; N <= 256)."""
    x, a_real, a_imag, B, C, D, gate = map(_f32, (x, a_real, a_imag, B, C, D, gate))
    M, L = x.shape
    N = a_real.shape[0]
    assert N <= 256
    y = np.empty((L, M), np.float32)
    U = np.empty((L, N), np.float32)
    H = np.empty((L, N), np.float32)
    lib().oracle_s4_ref_fwd_omp(M, N, L, dt, _ptr(x), _ptr(a_real), _ptr(a_imag), _ptr(B), _ptr(C),
                                _ptr(D), _ptr(gate), _ptr(y), _ptr(U), _ptr(H), int(threads))
    return y


def ssm_mamba_fwd(X, delta_proj, a_real, a_imag, B, C, D, gate, dt=0.1):
    X, delta_proj, a_real, a_imag, B, C, D, gate = map(_f32, (X, delta_proj, a_real, a_imag, B, C, D, gate))
    M = X.shape[0]
    N = a_real.shape[0]
    y = np.empty((M, M), np.float32)
    work = np.empty(M * M + 3 * N + M, np.float32)
    lib().oracle_ssm_mamba_fwd(M, N, dt, _ptr(X), _ptr(delta_proj), _ptr(a_real), _ptr(a_imag),
                               _ptr(B), _ptr(C), _ptr(D), _ptr(gate), _ptr(y), _ptr(work))
    return y


def selective_scan(u, delta, A, B, C, D=None, z=None, dt_bias=None, delta_softplus=True,
                   init_state=None, return_last_state=False, f64=False):
    """u, delta, z: [Bt, L, Dd]; A [Dd, N]; B, C [Bt, L, N]; D, dt_bias [Dd]."""
    u, delta, A, B, C, D, z, dt_bias, init_state = map(_f32, (u, delta, A, B, C, D, z, dt_bias, init_state))
    Bt, L, Dd = u.shape
    N = A.shape[1]
    if f64:
        out = np.empty((Bt, L, Dd), np.float64)
        last = np.empty((Bt, Dd, N), np.float64) if return_last_state else None
        fn = lib().oracle_selective_scan_f64
    else:
        out = np.empty((Bt, L, Dd), np.float32)
        last = np.empty((Bt, Dd, N), np.float32) if return_last_state else None
        fn = lib().oracle_selective_scan
    fn(Bt, L, Dd, N, int(bool(delta_softplus)), _ptr(u), _ptr(delta), _ptr(A), _ptr(B), _ptr(C),
       _ptr(D), _ptr(z), _ptr(dt_bias), _ptr(out), _ptr(init_state), _ptr(last))
    return (out, last) if return_last_state else out


def selective_state_update(state, u, delta, A, B, C, D=None, z=None, dt_bias=None, delta_softplus=True):
    """One decode step; returns (out [Bt, Dd], new_state [Bt, Dd, N])."""
    state = np.array(state, dtype=np.float32, copy=True)
    u, delta, A, B, C, D, z, dt_bias = map(_f32, (u, delta, A, B, C, D, z, dt_bias))
    Bt, Dd = u.shape
    N = A.shape[1]
    out = np.empty((Bt, Dd), np.float32)
    lib().oracle_selective_state_update(Bt, Dd, N, int(bool(delta_softplus)), _ptr(state), _ptr(u),
                                        _ptr(delta), _ptr(A), _ptr(B), _ptr(C), _ptr(D), _ptr(z),
                                        _ptr(dt_bias), _ptr(out))
    return out, state


def selective_scan_omp(u, delta, A, B, C, D=None, z=None, dt_bias=None, delta_softplus=True,
                       init_state=None, return_last_state=False, threads=0):
    """selective_scan's values bit for bit, (batch, 16-channel block) tasks over threads."""
    u, delta, A, B, C, D, z, dt_bias, init_state = map(_f32, (u, delta, A, B, C, D, z, dt_bias, init_state))
    Bt, L, Dd = u.shape
    N = A.shape[1]
    assert N <= 256
    out = np.empty((Bt, L, Dd), np.float32)
    last = np.empty((Bt, Dd, N), np.float32) if return_last_state else None
    lib().oracle_selective_scan_omp(Bt, L, Dd, N, int(bool(delta_softplus)), _ptr(u), _ptr(delta),
                                    _ptr(A), _ptr(B), _ptr(C), _ptr(D), _ptr(z), _ptr(dt_bias),
                                    _ptr(out), _ptr(init_state), _ptr(last), int(threads))
    return (out, last) if return_last_state else out


def selective_state_update_omp(state, u, delta, A, B, C, D=None, z=None, dt_bias=None,
                               delta_softplus=True, threads=0):
    """selective_state_update over threads; returns (out [Bt, Dd], new_state [Bt, Dd, N])."""
    state = np.array(state, dtype=np.float32, copy=True)
    u, delta, A, B, C, D, z, dt_bias = map(_f32, (u, delta, A, B, C, D, z, dt_bias))
    Bt, Dd = u.shape
    N = A.shape[1]
    assert N <= 256
    out = np.empty((Bt, Dd), np.float32)
    lib().oracle_selective_state_update_omp(Bt, Dd, N, int(bool(delta_softplus)), _ptr(state), _ptr(u),
                                            _ptr(delta), _ptr(A), _ptr(B), _ptr(C), _ptr(D), _ptr(z),
                                            _ptr(dt_bias), _ptr(out), int(threads))
    return out, state


def linear_omp(X, W, bias=None, act=0, threads=0):
    """linear's values bit for bit: a blocked product over a packed W^T (hx_oracle_omp.c)."""
    X, W, bias = _f32(X), _f32(W), _f32(bias)
    R, IN = X.shape
    OUT = W.shape[0]
    Y = np.empty((R, OUT), np.float32)
    Wt = np.empty((IN, OUT), np.float32)
    lib().oracle_linear_omp(R, IN, OUT, _ptr(X), _ptr(W), _ptr(bias), act, _ptr(Y), _ptr(Wt), int(threads))
    return Y


def r_linear(X, W, bias=None):
    """Linear::forward in the reference's execution shape (transpose copy, ijk matmul, broadcast
    bias add, hx_oracle_ref.c); linear's values bit for bit."""
    X, W, bias = _f32(X), _f32(W), _f32(bias)
    R, IN = X.shape
    OUT = W.shape[0]
    Y = np.empty((R, OUT), np.float32)
    lib().oracle_r_linear(R, IN, OUT, _ptr(X), _ptr(W), _ptr(bias), _ptr(Y))
    return Y


def conv1d_silu_omp(x, w, bias=None, threads=0):
    """conv1d_silu's values bit for bit, rows over threads."""
    x = np.asarray(x, np.float32)
    Bt, L, Dd = x.shape
    xs = np.ascontiguousarray(x)
    w, bias = _f32(w), _f32(bias)
    y = np.empty((Bt, L, Dd), np.float32)
    lib().oracle_conv1d_silu_omp(Bt, L, Dd, w.shape[1], _ptr(xs), Dd, _ptr(w), _ptr(bias), _ptr(y),
                                 int(threads))
    return y


def rmsnorm_omp(X, w, eps, threads=0):
    """rmsnorm's values bit for bit, rows over threads."""
    X, w = _f32(X), _f32(w)
    R, Dm = X.shape
    Y = np.empty_like(X)
    lib().oracle_rmsnorm_omp(R, Dm, _ptr(X), _ptr(w), eps, _ptr(Y), int(threads))
    return Y


def s4d_complex_omp(x, dt, a_re, a_im, B_re, B_im, C_re, C_im, D=None, threads=0):
    """s4d_complex in f32 arithmetic over threads (within rounding of the f64 checker)."""
    x, dt, a_re, a_im, B_re, B_im, C_re, C_im, D = map(_f32, (x, dt, a_re, a_im, B_re, B_im, C_re, C_im, D))
    Bt, L, Dd = x.shape
    N = a_re.shape[1]
    assert N <= 256
    y = np.empty((Bt, L, Dd), np.float32)
    lib().oracle_s4d_complex_omp(Bt, L, Dd, N, _ptr(x), _ptr(dt), _ptr(a_re), _ptr(a_im), _ptr(B_re),
                                 _ptr(B_im), _ptr(C_re), _ptr(C_im), _ptr(D), _ptr(y), int(threads))
    return y


class _Prims:
    """The primitives a composition (mamba_block, the byte LM) runs on.
    impl "seq": the sequential C restatement; "omp": hx_oracle_omp.c over `threads` threads (same
    values); "ref": Linear in the reference's execution shape (hx_oracle_ref.c), the rest
    sequential (the reference has no conv, scan or norm kernels of its own to time)."""

    def __init__(self, impl="seq", threads=0):
        assert impl in ("seq", "omp", "ref"), impl
        self.impl, self.threads = impl, threads

    def linear(self, X, W):
        if self.impl == "omp":
            return linear_omp(X, W, threads=self.threads)
        return r_linear(X, W) if self.impl == "ref" else linear(X, W)

    def conv1d_silu(self, x, w, b):
        return conv1d_silu_omp(x, w, b, self.threads) if self.impl == "omp" else conv1d_silu(x, w, b)

    def rmsnorm(self, X, w, eps):
        return rmsnorm_omp(X, w, eps, self.threads) if self.impl == "omp" else rmsnorm(X, w, eps)

    def scan(self, *a, **k):
        if self.impl == "omp":
            return selective_scan_omp(*a, **k, threads=self.threads)
        return selective_scan(*a, **k)

    def state_update(self, *a, **k):
        if self.impl == "omp":
            return selective_state_update_omp(*a, **k, threads=self.threads)
        return selective_state_update(*a, **k)


def r_s4_forward_ssm(x, a_real, a_imag, B, C, D, delta=None, lam=None, dt=0.1):
    """S4Block::forward_ssm in the reference's execution shape (hx_oracle_ref.c): x [M, L] ->
    y memory [L, M]; same values as s4_ref_fwd, bit for bit."""
    x, a_real, a_imag, B, C, D = map(_f32, (x, a_real, a_imag, B, C, D))
    M, L = x.shape
    N = a_real.shape[0]
    delta = _f32(delta) if delta is not None else np.zeros(M, np.float32)
    lam = _f32(lam) if lam is not None else np.zeros(N, np.float32)
    y = np.empty((L, M), np.float32)
    lib().oracle_r_s4_forward_ssm(M, N, L, dt, _ptr(x), _ptr(a_real), _ptr(a_imag), _ptr(B),
                                  _ptr(C), _ptr(D), _ptr(delta), _ptr(lam), _ptr(y))
    return y


def r_mamba_mlp(X, Wg, bg, Wo, bo):
    """Exported MambaBlock::forward_mamba in the reference's execution shape (hx_oracle_ref.c);
    same values as mamba_mlp, bit for bit."""
    X, Wg, bg, Wo, bo = map(_f32, (X, Wg, bg, Wo, bo))
    R, dm = X.shape
    di = Wg.shape[0]
    Y = np.empty((R, dm), np.float32)
    lib().oracle_r_mamba_mlp(R, dm, di, _ptr(X), _ptr(Wg), _ptr(bg), _ptr(Wo), _ptr(bo), _ptr(Y))
    return Y


def max_threads() -> int:
    return lib().oracle_max_threads()


def s4d_complex(x, dt, a_re, a_im, B_re, B_im, C_re, C_im, D=None):
    x, dt, a_re, a_im, B_re, B_im, C_re, C_im, D = map(_f32, (x, dt, a_re, a_im, B_re, B_im, C_re, C_im, D))
    Bt, L, Dd = x.shape
    N = a_re.shape[1]
    y = np.empty((Bt, L, Dd), np.float64)
    lib().oracle_s4d_complex(Bt, L, Dd, N, _ptr(x), _ptr(dt), _ptr(a_re), _ptr(a_im), _ptr(B_re),
                             _ptr(B_im), _ptr(C_re), _ptr(C_im), _ptr(D), _ptr(y))
    return y


def conv1d_silu(x, w, bias=None):
    """x [Bt, L, Dd] (any row stride), w [Dd, W], bias [Dd] -> y [Bt, L, Dd] float32."""
    x = np.asarray(x, np.float32)
    Bt, L, Dd = x.shape
    xs = np.ascontiguousarray(x)
    w, bias = _f32(w), _f32(bias)
    y = np.empty((Bt, L, Dd), np.float32)
    lib().oracle_conv1d_silu(Bt, L, Dd, w.shape[1], _ptr(xs), Dd, _ptr(w), _ptr(bias), _ptr(y))
    return y


def bf16_round(a):
    """Round-to-nearest-even to bfloat16, returned as float32 (the GPU path's storage format)."""
    a = np.ascontiguousarray(a, np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    out = r.astype(np.uint32).view(np.float32)
    return np.where(np.isnan(a), a, out)


def mamba_block(x, w_in, conv_w, conv_b, w_x, w_dt, dt_bias, A, D, w_out, dt_rank, bf16=True,
                round_out=True, return_state=False, impl="seq", threads=0):
    """Mamba block forward: x [Bt, L, d_model] -> [Bt, L, d_model].
    in_proj -> (x | z); SiLU(conv1d(x)); x_proj -> (dt_lo | B | C); dt = dt_lo . w_dt^T;
    selective_scan(softplus(dt + dt_bias)); out_proj. Every intermediate the GPU stores in bf16 is
    rounded to bf16 here too (``bf16=True``); arithmetic is f32. ``round_out=False`` leaves the
    out_proj result in f32 (the layer form, which adds it to an f32 residual stream).
    ``return_state``: also return the decode hand-off (scan last state [Bt, d_inner, N], conv
    window [Bt, d_conv-1, d_inner] = the last d_conv-1 conv inputs). ``impl``/``threads`` pick
    the primitives (_Prims: sequential, OpenMP or the reference's Linear); the values do not
    depend on them."""
    ops = _Prims(impl, threads)
    rnd = bf16_round if bf16 else (lambda a: np.asarray(a, np.float32))
    Bt, L, dm = x.shape
    di = w_dt.shape[0]
    N = A.shape[1]
    K = conv_w.shape[1]
    X = rnd(x).reshape(Bt * L, dm)
    xz = ops.linear(X, rnd(w_in))
    xp = rnd(xz[:, :di]).reshape(Bt, L, di)
    z = rnd(xz[:, di:]).reshape(Bt, L, di)
    xc = rnd(ops.conv1d_silu(xp, conv_w, conv_b))
    dbc = ops.linear(xc.reshape(Bt * L, di), rnd(w_x))
    dtlo = rnd(dbc[:, :dt_rank])
    Bm = rnd(dbc[:, dt_rank:dt_rank + N]).reshape(Bt, L, N)
    Cm = rnd(dbc[:, dt_rank + N:]).reshape(Bt, L, N)
    dt = rnd(ops.linear(dtlo, rnd(w_dt))).reshape(Bt, L, di)
    y, last = ops.scan(xc, dt, A, Bm, Cm, D, z, dt_bias, True, return_last_state=True)
    out = ops.linear(rnd(y).reshape(Bt * L, di), rnd(w_out))
    out = (rnd(out) if round_out else out).reshape(Bt, L, dm)
    if not return_state:
        return out
    conv = np.zeros((Bt, max(K - 1, 1), di), np.float32)
    for j in range(K - 1):
        t = L - (K - 1) + j
        if t >= 0:
            conv[:, j, :] = xp[:, t, :]
    return out, last, conv


def conv1d_step(x, w, bias, state):
    """One recurrent conv step: x [Bt, Dd]; state [Bt, W-1, Dd] (copied, returned advanced)."""
    x = np.asarray(x, np.float32)
    w = np.asarray(w, np.float32)
    W = w.shape[1]
    win = np.concatenate([np.asarray(state, np.float32)[:, :W - 1, :], x[:, None, :]], axis=1)
    xc = np.empty(x.shape, np.float32)
    # same op order as oracle_conv1d_silu: bias, then taps j ascending
    acc = np.broadcast_to(np.asarray(bias, np.float32), x.shape).astype(np.float32) if bias is not None \
        else np.zeros(x.shape, np.float32)
    for j in range(W):
        acc = (acc + w[:, j][None, :] * win[:, j, :]).astype(np.float32)
    xc[:] = silu(acc)
    new_state = win[:, 1:, :].copy() if W > 1 else np.asarray(state, np.float32).copy()
    return xc, new_state


def mamba_layer_decode(resid, p, state, dt_rank, eps, bf16=True, impl="seq", threads=0):
    """One decode step of a pre-norm layer; resid [Bt, d_model] f32. Returns (resid, state)."""
    ops = _Prims(impl, threads)
    rnd = bf16_round if bf16 else (lambda a: np.asarray(a, np.float32))
    ssm_st, conv_st = state
    di = p["w_dt"].shape[0]
    N = p["A"].shape[1]
    xn = rnd(ops.rmsnorm(resid, p["norm_w"], eps))
    xz = ops.linear(xn, rnd(p["w_in"]))
    xp, z = rnd(xz[:, :di]), rnd(xz[:, di:])
    xc, conv_st = conv1d_step(xp, p["conv_w"], p["conv_b"], conv_st)
    xc = rnd(xc)
    dbc = ops.linear(xc, rnd(p["w_x"]))
    dtlo = rnd(dbc[:, :dt_rank])
    Bv, Cv = rnd(dbc[:, dt_rank:dt_rank + N]), rnd(dbc[:, dt_rank + N:])
    dt = rnd(ops.linear(dtlo, rnd(p["w_dt"])))
    y, ssm_st = ops.state_update(ssm_st, xc, dt, p["A"], Bv, Cv, p["D"], z, p["dt_bias"], True)
    resid = (resid + ops.linear(rnd(y), rnd(p["w_out"]))).astype(np.float32)
    return resid, (ssm_st, conv_st)


def lm_head(x, params, eps, bf16=True, impl="seq", threads=0):
    ops = _Prims(impl, threads)
    rnd = bf16_round if bf16 else (lambda a: np.asarray(a, np.float32))
    shp = x.shape
    xn = rnd(ops.rmsnorm(x.reshape(-1, shp[-1]), params["norm_f"], eps))
    return ops.linear(xn, rnd(params["w_head"])).reshape(*shp[:-1], -1)


def lm_prefill(tokens, params, dt_rank, eps=1e-5, bf16=True, impl="seq", threads=0):
    """Byte LM prefill: tokens [Bt, L] int -> (logits [Bt, L, vocab] f32, per-layer state).
    bf16=False keeps every intermediate in f32 (the CPU timing legs); impl/threads as in
    mamba_block."""
    rnd = bf16_round if bf16 else (lambda a: np.asarray(a, np.float32))
    ops = _Prims(impl, threads)
    x = np.asarray(params["embed"], np.float32)[np.asarray(tokens)]
    Bt, L, dm = x.shape
    states = []
    for p in params["layers"]:
        xn = rnd(ops.rmsnorm(x.reshape(-1, dm), p["norm_w"], eps)).reshape(Bt, L, dm)
        blk = {k: p[k] for k in ("w_in", "conv_w", "conv_b", "w_x", "w_dt", "dt_bias", "A", "D", "w_out")}
        out, last, conv = mamba_block(xn, **blk, dt_rank=dt_rank, bf16=bf16, round_out=False,
                                      return_state=True, impl=impl, threads=threads)
        x = (x + out).astype(np.float32)
        states.append((last, conv))
    return lm_head(x, params, eps, bf16, impl, threads), states


def lm_decode_step(tokens, params, states, dt_rank, eps=1e-5, bf16=True, impl="seq", threads=0):
    """One decode step: tokens [Bt] -> (logits [Bt, vocab], new per-layer states)."""
    x = np.asarray(params["embed"], np.float32)[np.asarray(tokens)]
    new = []
    for p, st in zip(params["layers"], states):
        x, st = mamba_layer_decode(x, p, st, dt_rank, eps, bf16, impl, threads)
        new.append(st)
    return lm_head(x, params, eps, bf16, impl, threads), new


# ------------------------------------------------------------------ independent float64 restatements

def numpy_selective_scan(u, delta, A, B, C, D=None, z=None, dt_bias=None, delta_softplus=True,
                         init_state=None):
    """Vectorised over (batch, channel, state), float64; returns (out, last_state)."""
    u = np.asarray(u, np.float64)
    dl = np.asarray(delta, np.float64)
    if dt_bias is not None:
        dl = dl + np.asarray(dt_bias, np.float64)[None, None, :]
    if delta_softplus:
        dl = np.where(dl > 20.0, dl, np.log1p(np.exp(np.minimum(dl, 20.0))))
    A = np.asarray(A, np.float64)
    B = np.asarray(B, np.float64)
    C = np.asarray(C, np.float64)
    Bt, L, Dd = u.shape
    N = A.shape[1]
    h = np.zeros((Bt, Dd, N)) if init_state is None else np.asarray(init_state, np.float64).copy()
    out = np.empty((Bt, L, Dd))
    for t in range(L):
        dA = np.exp(dl[:, t, :, None] * A[None])                          # [Bt, Dd, N]
        h = dA * h + (dl[:, t, :] * u[:, t, :])[:, :, None] * B[:, t, None, :]
        y = np.einsum("bdn,bn->bd", h, C[:, t, :])
        if D is not None:
            y = y + np.asarray(D, np.float64)[None] * u[:, t, :]
        if z is not None:
            zz = np.asarray(z, np.float64)[:, t, :]
            y = y * zz / (1.0 + np.exp(-zz))
        out[:, t, :] = y
    return out, h


def numpy_s4_ref(x, a_real, a_imag, B, C, D, gate=None, dt=0.1):
    """float64 restatement of S4Block::forward_ssm (ssm.rs:138-186); y memory [L, M]."""
    x = np.asarray(x, np.float64)
    M, L = x.shape
    a = np.exp(np.asarray(a_real, np.float64) * dt) * np.cos(np.asarray(a_imag, np.float64) * dt)
    Bd = np.asarray(B, np.float64) * dt
    C = np.asarray(C, np.float64)
    D = np.asarray(D, np.float64)
    h = np.zeros(a.shape[0])
    y = np.empty((L, M))
    for t in range(L):
        h = a * h + Bd @ x[:, t]
        y[t] = C @ h + D * x[:, t]
    if gate is not None:
        y = y * np.asarray(gate, np.float64)[None, :]
    return y


def numpy_conv1d_silu(x, w, bias=None):
    """float64: per-channel full np.convolve with the reversed taps, first L outputs."""
    x = np.asarray(x, np.float64)
    w = np.asarray(w, np.float64)
    Bt, L, Dd = x.shape
    y = np.empty((Bt, L, Dd))
    for b in range(Bt):
        for d in range(Dd):
            # causal: y[t] = sum_j w[j] x[t-W+1+j] == (x * w[::-1])[t] of the full convolution
            y[b, :, d] = np.convolve(x[b, :, d], w[d, ::-1])[:L]
    if bias is not None:
        y = y + np.asarray(bias, np.float64)[None, None, :]
    return y / (1.0 + np.exp(-y))


def numpy_mamba_block(x, w_in, conv_w, conv_b, w_x, w_dt, dt_bias, A, D, w_out, dt_rank,
                      round_out=True, return_state=False, return_terms=False):
    """float64 block with the same bf16 storage rounding points as ``mamba_block`` (and its
    ``round_out`` / ``return_state`` options). ``return_terms``: also return |y| . |w_out|^T
    [Bt, L, d_model], the sum of the magnitudes of the terms the output product adds (the scale
    a componentwise error bound of that product is relative to)."""
    r = lambda a: bf16_round(np.asarray(a, np.float32)).astype(np.float64)  # noqa: E731
    Bt, L, dm = x.shape
    di = w_dt.shape[0]
    N = A.shape[1]
    K = np.asarray(conv_w).shape[1]
    xz = r(x).reshape(-1, dm) @ r(w_in).T
    xp, z = r(xz[:, :di]).reshape(Bt, L, di), r(xz[:, di:]).reshape(Bt, L, di)
    xc = r(numpy_conv1d_silu(xp, conv_w, conv_b))
    dbc = xc.reshape(-1, di) @ r(w_x).T
    dtlo = r(dbc[:, :dt_rank])
    Bm = r(dbc[:, dt_rank:dt_rank + N]).reshape(Bt, L, N)
    Cm = r(dbc[:, dt_rank + N:]).reshape(Bt, L, N)
    dt = r(dtlo @ r(w_dt).T).reshape(Bt, L, di)
    y, last = numpy_selective_scan(xc, dt, A, Bm, Cm, D, z, dt_bias, True)
    out = r(y).reshape(-1, di) @ r(w_out).T
    out = (r(out) if round_out else out).reshape(Bt, L, dm)
    if return_terms:
        terms = (np.abs(r(y)).reshape(-1, di) @ np.abs(r(w_out)).T).reshape(Bt, L, dm)
        return (out, terms) if not return_state else (out, last, conv, terms)
    if not return_state:
        return out
    conv = np.zeros((Bt, max(K - 1, 1), di))
    for j in range(K - 1):
        t = L - (K - 1) + j
        if t >= 0:
            conv[:, j, :] = xp[:, t, :]
    return out, last, conv


def numpy_rmsnorm(X, w, eps):
    """float64 RMSNorm (crates/nn/src/lib.rs:258-285): x / sqrt(mean(x^2) + eps) * w per row."""
    X = np.asarray(X, np.float64)
    return X / np.sqrt((X * X).mean(axis=-1, keepdims=True) + eps) * np.asarray(w, np.float64)


def numpy_lm_head(x, params, eps, return_terms=False):
    """float64 head: logits = bf16(RMSNorm(x)) . w_head^T. ``return_terms``: also |xn| . |w_head|^T,
    the sum of the magnitudes of the terms each logit adds (the scale of a componentwise bound)."""
    r = lambda a: bf16_round(np.asarray(a, np.float32)).astype(np.float64)  # noqa: E731
    shp = x.shape
    xn = r(numpy_rmsnorm(np.asarray(x, np.float64).reshape(-1, shp[-1]), params["norm_f"], eps))
    w = r(params["w_head"])
    logits = (xn @ w.T).reshape(*shp[:-1], -1)
    if not return_terms:
        return logits
    return logits, (np.abs(xn) @ np.abs(w).T).reshape(*shp[:-1], -1)


def numpy_lm_prefill(tokens, params, dt_rank, eps=1e-5, return_terms=False):
    """float64 twin of ``lm_prefill`` with the same bf16 storage rounding points: the exact value
    of what the f32 restatement computes, for bounding its own rounding. ``return_terms``: also
    the head's term magnitudes (numpy_lm_head)."""
    r = lambda a: bf16_round(np.asarray(a, np.float32)).astype(np.float64)  # noqa: E731
    x = np.asarray(params["embed"], np.float64)[np.asarray(tokens)]
    Bt, L, dm = x.shape
    states = []
    for p in params["layers"]:
        xn = r(numpy_rmsnorm(x.reshape(-1, dm), p["norm_w"], eps)).reshape(Bt, L, dm)
        blk = {k: p[k] for k in ("w_in", "conv_w", "conv_b", "w_x", "w_dt", "dt_bias", "A", "D", "w_out")}
        out, last, conv = numpy_mamba_block(xn, **blk, dt_rank=dt_rank, round_out=False, return_state=True)
        x = x + out
        states.append((last, conv))
    if return_terms:
        logits, terms = numpy_lm_head(x, params, eps, return_terms=True)
        return logits, states, terms
    return numpy_lm_head(x, params, eps), states


def numpy_lm_decode_step(tokens, params, states, dt_rank, eps=1e-5, return_terms=False):
    """float64 twin of ``lm_decode_step`` (same bf16 storage rounding points); ``return_terms`` as
    numpy_lm_prefill's."""
    r = lambda a: bf16_round(np.asarray(a, np.float32)).astype(np.float64)  # noqa: E731
    x = np.asarray(params["embed"], np.float64)[np.asarray(tokens)]
    new = []
    for p, (ssm_st, conv_st) in zip(params["layers"], states):
        di = p["w_dt"].shape[0]
        N = np.asarray(p["A"]).shape[1]
        w = np.asarray(p["conv_w"], np.float64)
        K = w.shape[1]
        xn = r(numpy_rmsnorm(x, p["norm_w"], eps))
        xz = xn @ r(p["w_in"]).T
        xp, z = r(xz[:, :di]), r(xz[:, di:])
        win = np.concatenate([np.asarray(conv_st, np.float64)[:, :K - 1, :], xp[:, None, :]], axis=1)
        acc = np.asarray(p["conv_b"], np.float64)[None, :] + np.einsum("dj,bjd->bd", w, win)
        xc = r(acc / (1.0 + np.exp(-acc)))
        conv_st = win[:, 1:, :] if K > 1 else np.asarray(conv_st, np.float64)
        dbc = xc @ r(p["w_x"]).T
        dtlo = r(dbc[:, :dt_rank])
        Bv, Cv = r(dbc[:, dt_rank:dt_rank + N]), r(dbc[:, dt_rank + N:])
        dt = r(dtlo @ r(p["w_dt"]).T)
        y, ssm_st = numpy_selective_scan(xc[:, None], dt[:, None], p["A"], Bv[:, None], Cv[:, None], p["D"],
                                         z[:, None], p["dt_bias"], True, init_state=ssm_st)
        x = x + r(y[:, 0]) @ r(p["w_out"]).T
        new.append((ssm_st, conv_st))
    if return_terms:
        logits, terms = numpy_lm_head(x, params, eps, return_terms=True)
        return logits, new, terms
    return numpy_lm_head(x, params, eps), new


# ------------------------------------------------------------------ tensor primitives
# Restatements of CpuTensor's primitives (crates/backend-cpu/src/lib.rs) that HipTensor's
# device primitives (hx_binary_f32, hx_unary_f32, hx_mean_axis_f32, hx_copy_strided_f32) are
# checked against. Elementwise add/sub/mul/div are single IEEE float32 operations, so numpy's
# float32 arithmetic is their restatement.

UNARY = {"exp": 0, "cos": 1, "sin": 2, "sqrt": 3, "silu": 4, "neg": 5, "mul_scalar": 6,
         "add_scalar": 7, "abs": 8, "log": 9, "sigmoid": 10}


def unary(op, x, s=0.0):
    """libm maps of CpuTensor (lib.rs:768-932, 1154-1178); op as in UNARY."""
    x = _f32(x)
    y = np.empty_like(x)
    lib().oracle_unary(UNARY[op], x.size, _ptr(x), s, _ptr(y))
    return y


def mean_axis(x, axis):
    """ndarray 0.15 mean_axis (TensorReduce::mean of one axis, lib.rs:995-1010) of a row-major
    array, with ndarray's summation order (the lane fold on the last axis)."""
    x = _f32(x)
    d = x.shape
    outer = int(np.prod(d[:axis], dtype=np.int64))
    inner = int(np.prod(d[axis + 1:], dtype=np.int64))
    y = np.empty(d[:axis] + d[axis + 1:], np.float32)
    lane = 1 if axis == len(d) - 1 else 0
    lib().oracle_mean_axis(outer, d[axis], inner, lane, _ptr(x), _ptr(y))
    return y


def rmsnorm_ref(X, w, eps):
    """nn::RMSNorm::forward (lib.rs:258-285) in its primitives' order (eps' = eps)."""
    X, w = _f32(X), _f32(w)
    R, Dm = X.shape
    Y = np.empty_like(X)
    work = np.empty(Dm, np.float32)
    lib().oracle_rmsnorm_ref(R, Dm, _ptr(X), _ptr(w), eps, _ptr(Y), _ptr(work))
    return Y


def _row_major_strides(dims):
    s = [1] * len(dims)
    for i in range(len(dims) - 1, 0, -1):
        s[i - 1] = s[i] * dims[i]
    return s


def broadcast_to(x, shape):
    """CpuTensor::broadcast_to (lib.rs:1352-1518): the (1,2) / (2,3) / (1,3) cases, and the
    generic index map of lib.rs:511-560 as written for every other rank pair (target dim j reads
    the source with the source's own stride at index j, 1 past its rank). Raises ValueError where
    the reference returns ShapeMismatch."""
    x = np.asarray(x, np.float32)
    s, t = list(x.shape), list(shape)
    if len(s) > len(t):
        raise ValueError("ShapeMismatch")
    if s == t:
        return x.copy()
    padded = [1] * (len(t) - len(s)) + s
    for pd, td in zip(padded, t):
        if pd != 1 and pd != td:
            raise ValueError("ShapeMismatch")
    flat = x.reshape(-1)
    if (len(s), len(t)) == (1, 2):
        if s[0] == t[1]:
            return np.tile(flat, (t[0], 1))
        if s[0] == t[0]:
            return np.repeat(flat, t[1]).reshape(t)
        raise ValueError("ShapeMismatch")
    if (len(s), len(t)) == (2, 3):
        if s == t[1:] or (s[0] == 1 and s[1] == t[2]):
            return np.broadcast_to(x, t).copy()
        raise ValueError("ShapeMismatch")
    if (len(s), len(t)) == (1, 3):
        if s[0] == t[2]:
            return np.broadcast_to(x, t).copy()
        raise ValueError("ShapeMismatch")
    ss = _row_major_strides(s)
    out = np.empty(int(np.prod(t, dtype=np.int64)), np.float32)
    for i in range(out.size):   # small cases only: the reference's loop, element by element
        idx, rem = 0, i
        for j in range(len(t) - 1, -1, -1):
            c = rem % t[j]
            rem //= t[j]
            sc = c % padded[j] if padded[j] != 1 else 0
            idx += sc * (ss[j] if j < len(ss) else 1)
        out[i] = flat[idx]
    return out.reshape(t)


def stack(tensors, dim):
    """CpuTensor::stack (lib.rs:254-335, generic 390-467): returns (data, shape field). For 1..3-D
    inputs the data are the inputs back to back whatever `dim`; the shape field inserts the count
    at `dim`. Other ranks: a true stack along `dim`."""
    arrs = [np.asarray(a, np.float32) for a in tensors]
    if len(arrs) == 1:
        return arrs[0].copy(), list(arrs[0].shape)
    shape = list(arrs[0].shape)
    field = shape[:dim] + [len(arrs)] + shape[dim:]
    if 1 <= len(shape) <= 3:
        return np.concatenate([a.reshape(-1) for a in arrs]).reshape(field), field
    return np.stack(arrs, axis=dim), field


def transpose(x, d0, d1):
    """CpuTensor::transpose (lib.rs:115-137): logical axis swap."""
    return np.ascontiguousarray(np.swapaxes(np.asarray(x, np.float32), d0, d1))


def slice2d(x, start, end):
    """CpuTensor::slice of a 2-D tensor (lib.rs:158-175)."""
    return np.asarray(x, np.float32)[start[0]:end[0], start[1]:end[1]].copy()


def cat1d(tensors):
    """CpuTensor::cat of 1-D tensors (lib.rs:229-246)."""
    return np.concatenate([np.asarray(a, np.float32) for a in tensors])
