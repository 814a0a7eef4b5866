"""Pins the CPU oracle (oracle/hx_oracle.c) before anything is compared against it.

Each oracle function is checked against the reference's own known-answer tests where they exist
(backend-cpu/src/lib.rs:1733-1758), closed forms, invariants and an independent float64 numpy
restatement — chosen so a dropped term, a wrong sign/index or a transposed operand fails.
The planted-mistake tests at the end show the checks do fail on such mistakes.
"""
import numpy as np
import pytest

import oracle
from tests.util import norm_err, rel_err

F = np.float32


# ------------------------------------------------------------------ CpuTensor primitives

def test_reference_kat_matmul_ones():
    # backend-cpu/src/lib.rs:1747-1758: ones[2,3] . ones[3,4] == 3 everywhere (to 1e-6)
    y = oracle.matmul(np.ones((2, 3), F), np.ones((3, 4), F))
    assert y.shape == (2, 4)
    assert np.all(np.abs(y - 3.0) < 1e-6)


def test_reference_kat_linear_ones_plus_bias():
    # Linear with W = ones[4,3] (out, in) on ones[2,3]: 3 + bias (ones+ones == 2 KAT: lib.rs:1733-1744)
    y = oracle.linear(np.ones((2, 3), F), np.ones((4, 3), F), np.ones(4, F))
    assert np.all(y == 4.0)
    assert np.all(oracle.linear(np.ones((2, 3), F), np.zeros((4, 3), F), np.ones(4, F)) + 1.0 == 2.0)


def test_matmul_vs_numpy_f64():
    rng = np.random.default_rng(1)
    A = rng.standard_normal((17, 33), dtype=F)
    B = rng.standard_normal((33, 9), dtype=F)
    assert rel_err(oracle.matmul(A, B), A.astype(np.float64) @ B.astype(np.float64)) < 1e-4


def test_matmul_is_sequential_f32_ijk():
    # a value where summation order matters in f32: 1e8 + 1 - 1e8 (k ascending) == 0 in f32
    A = np.array([[1e8, 1.0, -1e8]], F)
    B = np.ones((3, 1), F)
    assert oracle.matmul(A, B)[0, 0] == np.float32(np.float32(np.float32(1e8) + 1.0) - np.float32(1e8))


def test_silu_closed_form():
    x = np.array([0.0, 1.0, -1.0, 30.0, -30.0, 5.5], F)
    y = oracle.silu(x)
    ref = x.astype(np.float64) / (1.0 + np.exp(-x.astype(np.float64)))
    assert y[0] == 0.0
    assert rel_err(y, ref) < 1e-6
    assert abs(y[3] - 30.0) < 1e-5


def test_linear_and_mlp_vs_numpy():
    rng = np.random.default_rng(2)
    X = rng.uniform(-1, 1, (10, 8)).astype(F)
    Wg = rng.standard_normal((16, 8), dtype=F)
    bg = rng.standard_normal(16, dtype=F)
    Wo = rng.standard_normal((8, 16), dtype=F)
    bo = rng.standard_normal(8, dtype=F)
    X64 = X.astype(np.float64)
    H = X64 @ Wg.T.astype(np.float64) + bg
    S = H / (1 + np.exp(-H))
    Y = S @ Wo.T.astype(np.float64) + bo
    assert rel_err(oracle.mamba_mlp(X, Wg, bg, Wo, bo), Y) < 1e-5


def test_rmsnorm_constant_rows():
    x = np.full((3, 8), 2.0, F)
    y = oracle.rmsnorm(x, np.ones(8, F), 1e-6)
    assert rel_err(y, np.full((3, 8), 2.0 / np.sqrt(4.0 + 1e-6))) < 1e-6
    rng = np.random.default_rng(3)
    x = rng.standard_normal((5, 32), dtype=F)
    w = rng.standard_normal(32, dtype=F)
    x64 = x.astype(np.float64)
    ref = x64 / np.sqrt((x64 ** 2).mean(-1, keepdims=True) + 1e-5) * w
    assert rel_err(oracle.rmsnorm(x, w, 1e-5), ref) < 1e-5


# ------------------------------------------------------------------ S4 reference mode

def s4_params(M, N, seed, a_real=None, a_imag=None, D=None):
    rng = np.random.default_rng(seed)
    return dict(
        a_real=np.zeros(N, F) if a_real is None else a_real.astype(F),
        a_imag=rng.standard_normal(N, dtype=F) if a_imag is None else a_imag.astype(F),
        B=(rng.standard_normal((N, M)) * 0.1).astype(F),
        C=(rng.standard_normal((M, N)) * 0.1).astype(F),
        D=rng.standard_normal(M, dtype=F) if D is None else D.astype(F),
    )


def test_s4_zero_input_zero_output():
    p = s4_params(6, 4, 0)
    y = oracle.s4_ref_fwd(np.zeros((6, 9), F), **p)
    assert y.shape == (9, 6) and np.all(y == 0)


def test_s4_impulse_response_closed_form():
    M, N, L, j = 5, 4, 12, 2
    p = s4_params(M, N, 1, a_real=np.full(4, -0.5), a_imag=np.pi * np.arange(4))
    x = np.zeros((M, L), F)
    x[j, 0] = 1.0
    y = oracle.s4_ref_fwd(x, **p)
    dt = 0.1
    a = np.exp(-0.5 * dt) * np.cos(np.pi * np.arange(N) * dt)
    Bd = p["B"].astype(np.float64) * dt
    for t in range(L):
        ref = p["C"].astype(np.float64) @ (a ** t * Bd[:, j])
        if t == 0:
            ref[j] += p["D"][j]
        assert rel_err(y[t], ref) < 1e-5, t


def test_s4_step_response_geometric_series():
    M, N, L, j = 4, 3, 40, 1
    p = s4_params(M, N, 2, a_real=np.array([-1.0, -2.0, -0.3]), a_imag=np.array([0.0, 3.0, 7.0]))
    x = np.zeros((M, L), F)
    x[j, :] = 1.0
    y = oracle.s4_ref_fwd(x, **p)
    dt = 0.1
    a = np.exp(p["a_real"] * dt) * np.cos(p["a_imag"] * dt)
    Bd = p["B"].astype(np.float64)[:, j] * dt
    for t in range(L):
        h = (1 - a ** (t + 1)) / (1 - a) * Bd
        ref = p["C"].astype(np.float64) @ h
        ref[j] += p["D"][j]
        assert rel_err(y[t], ref) < 1e-5


def test_s4_a_equal_one_is_prefix_sum():
    M, N, L = 6, 5, 30
    p = s4_params(M, N, 3, a_real=np.zeros(N), a_imag=np.zeros(N))
    x = np.random.default_rng(4).standard_normal((M, L)).astype(F)
    y = oracle.s4_ref_fwd(x, **p)
    H = np.cumsum((p["B"].astype(np.float64) * 0.1) @ x.astype(np.float64), axis=1)  # [N, L]
    ref = (p["C"].astype(np.float64) @ H).T + (p["D"][:, None] * x).T
    assert rel_err(y, ref) < 1e-5


def test_s4_b_zero_gives_feedthrough_and_gate():
    M, N, L = 7, 4, 11
    p = s4_params(M, N, 5)
    p["B"] = np.zeros_like(p["B"])
    x = np.random.default_rng(6).standard_normal((M, L)).astype(F)
    gate = np.random.default_rng(7).standard_normal(M).astype(F)
    y = oracle.s4_ref_fwd(x, gate=gate, **p)
    assert np.array_equal(y, ((p["D"][:, None] * x).T * gate[None, :]).astype(F))


def test_s4_linearity_and_numpy_bruteforce():
    M, N, L = 8, 4, 16
    p = s4_params(M, N, 8, a_real=np.full(N, -0.5), a_imag=np.pi * np.arange(N))
    rng = np.random.default_rng(9)
    x1 = rng.standard_normal((M, L)).astype(F)
    x2 = rng.standard_normal((M, L)).astype(F)
    y12 = oracle.s4_ref_fwd(x1 + 2 * x2, **p)
    assert rel_err(y12, oracle.s4_ref_fwd(x1, **p).astype(np.float64) + 2 * oracle.s4_ref_fwd(x2, **p)) < 1e-4
    assert rel_err(oracle.s4_ref_fwd(x1, **p), oracle.numpy_s4_ref(x1, **p)) < 1e-5


def test_ssm_mamba_is_matmul_then_s4_then_gate():
    M, N = 12, 4
    rng = np.random.default_rng(10)
    X = rng.standard_normal((M, M)).astype(F)
    dp = (rng.standard_normal((M, M)) * 0.1).astype(F)
    gate = (rng.standard_normal(M) * 0.1).astype(F)
    p = s4_params(M, N, 11)
    y = oracle.ssm_mamba_fwd(X, dp, gate=gate, **p)
    delta = oracle.matmul(X, dp)
    assert np.array_equal(y, oracle.s4_ref_fwd(delta, gate=gate, **p))
    ref = oracle.numpy_s4_ref(X.astype(np.float64) @ dp.astype(np.float64), gate=gate, **p)
    assert rel_err(y, ref) < 1e-4


# ------------------------------------------------------------------ selective scan

def inputs(bt, L, dim, N, seed, **kw):
    from tests.util import scan_inputs
    return scan_inputs(bt, L, dim, N, seed, **kw)


def test_scan_b_zero_is_gated_feedthrough():
    x = inputs(2, 9, 5, 4, 0)
    x["B"][:] = 0
    out = oracle.selective_scan(**x)
    u, z = x["u"].astype(np.float64), x["z"].astype(np.float64)
    assert rel_err(out, x["D"] * u * z / (1 + np.exp(-z))) < 1e-6
    x2 = inputs(2, 9, 5, 4, 0)
    x2["C"][:] = 0
    assert rel_err(oracle.selective_scan(**x2), x["D"] * u * z / (1 + np.exp(-z))) < 1e-6


def test_scan_a_zero_is_prefix_sum():
    x = inputs(2, 25, 6, 8, 1, with_z=False)
    x["A"][:] = 0
    out = oracle.selective_scan(**x)
    dl = x["delta"].astype(np.float64)
    dl = np.log1p(np.exp(dl))
    du = dl * x["u"]                                                     # [b, L, d]
    H = np.cumsum(du[..., None] * x["B"][:, :, None, :].astype(np.float64), axis=1)   # [b, L, d, n]
    ref = np.einsum("bldn,bln->bld", H, x["C"].astype(np.float64)) + x["D"] * x["u"]
    assert rel_err(out, ref) < 1e-5


def test_scan_dt_bias_inside_softplus_closed_form():
    """dt_bias enters softplus(delta + dt_bias). With A = 0 the state is a prefix sum, and with
    delta[b, t, d] = log(expm1(c[d])) - bias[d] the step size is exactly c[d] only if the bias is
    added inside the softplus: out = (C_t . c_d sum_{s<=t} u_s B_s + D u_t) silu(z_t). A bias
    dropped, applied after the softplus, or with the wrong sign misses by O(1)."""
    bt, L, dim, N = 2, 30, 4, 8
    x = inputs(bt, L, dim, N, 31)
    x["A"][:] = 0
    c = np.array([0.25, 0.5, 1.0, 2.0])                       # target step sizes per channel
    bias = np.array([-1.5, 0.0, 0.75, 3.0], F)
    x["dt_bias"] = bias
    x["delta"] = np.broadcast_to((np.log(np.expm1(c)) - bias).astype(F), (bt, L, dim)).copy()
    out = oracle.selective_scan(**x)
    u, z = x["u"].astype(np.float64), x["z"].astype(np.float64)
    H = np.cumsum(c[None, None, :, None] * u[..., None] * x["B"][:, :, None, :].astype(np.float64), axis=1)
    y = np.einsum("bldn,bln->bld", H, x["C"].astype(np.float64)) + x["D"] * u
    ref = y * z / (1 + np.exp(-z))
    assert rel_err(out, ref) < 1e-5
    # the planted mistakes this closed form catches (restated here on the CPU, not in the oracle)
    for wrong in (np.log1p(np.exp(x["delta"].astype(np.float64))),                 # bias dropped
                  np.log1p(np.exp(x["delta"].astype(np.float64))) + bias,          # bias after softplus
                  np.log1p(np.exp(x["delta"].astype(np.float64) - bias))):         # wrong sign
        Hw = np.cumsum(wrong[..., None] * u[..., None] * x["B"][:, :, None, :].astype(np.float64), axis=1)
        yw = (np.einsum("bldn,bln->bld", Hw, x["C"].astype(np.float64)) + x["D"] * u) * z / (1 + np.exp(-z))
        assert rel_err(out, yw) > 1e-2


def test_scan_dt_bias_without_softplus_is_added_to_delta():
    """delta_softplus off: dt = delta + dt_bias (no softplus), checked on the single-state
    geometric series with the bias carrying the whole step size (delta = 0)."""
    L, dl, A, u, Bv, Cv = 40, 0.3, -1.2, 0.8, 1.1, 0.7
    f = lambda v, shape: np.full(shape, v, F)
    out = oracle.selective_scan(f(u, (1, L, 1)), f(0.0, (1, L, 1)), f(A, (1, 1)), f(Bv, (1, L, 1)),
                                f(Cv, (1, L, 1)), dt_bias=f(dl, (1,)), delta_softplus=False)
    a = np.exp(dl * A)
    t = np.arange(L)
    assert rel_err(out[0, :, 0], Cv * dl * u * Bv * (1 - a ** (t + 1)) / (1 - a)) < 1e-5


def test_scan_single_state_geometric_series():
    L, dl, A, u, Bv, Cv = 50, 0.2, -1.5, 0.7, 1.3, -0.9
    f = lambda v, shape: np.full(shape, v, F)
    out = oracle.selective_scan(f(u, (1, L, 1)), f(dl, (1, L, 1)), f(A, (1, 1)), f(Bv, (1, L, 1)),
                                f(Cv, (1, L, 1)), delta_softplus=False)
    a = np.exp(dl * A)
    t = np.arange(L)
    ref = Cv * dl * u * Bv * (1 - a ** (t + 1)) / (1 - a)
    assert rel_err(out[0, :, 0], ref) < 1e-5


def test_scan_split_sequence_equals_whole():
    x = inputs(2, 40, 7, 16, 2, with_bias=True)
    out, last = oracle.selective_scan(**x, return_last_state=True)
    k = 17
    first = {n: (v[:, :k] if n in ("u", "delta", "B", "C", "z") else v) for n, v in x.items()}
    second = {n: (v[:, k:] if n in ("u", "delta", "B", "C", "z") else v) for n, v in x.items()}
    o1, s1 = oracle.selective_scan(**first, return_last_state=True)
    o2, s2 = oracle.selective_scan(**second, init_state=s1, return_last_state=True)
    assert np.array_equal(np.concatenate([o1, o2], 1), out)
    assert np.array_equal(s2, last)


def test_scan_decode_steps_equal_prefill():
    x = inputs(3, 12, 5, 16, 3)
    out, last = oracle.selective_scan(**x, return_last_state=True)
    state = np.zeros((3, 5, 16), F)
    for t in range(12):
        o, state = oracle.selective_state_update(state, x["u"][:, t], x["delta"][:, t], x["A"],
                                                 x["B"][:, t], x["C"][:, t], x["D"], x["z"][:, t])
        assert np.array_equal(o, out[:, t])
    assert np.array_equal(state, last)


def test_scan_f32_f64_and_numpy_agree():
    x = inputs(2, 300, 9, 16, 4, with_bias=True, s4d_real_A=False)
    o32 = oracle.selective_scan(**x)
    o64, s64 = oracle.selective_scan(**x, f64=True, return_last_state=True)
    on, sn = oracle.numpy_selective_scan(**x)
    assert rel_err(on, o64) < 1e-10
    assert rel_err(sn, s64) < 1e-10
    assert rel_err(o32, o64) < 1e-4


def test_scan_omp_matches_serial():
    # 33 channels: two full 16-channel tasks and a ragged one per batch row
    x = inputs(2, 64, 33, 16, 5)
    assert np.array_equal(oracle.selective_scan_omp(**x, threads=3), oracle.selective_scan(**x))
    init = np.random.default_rng(6).standard_normal((2, 33, 16)).astype(F)
    o, s = oracle.selective_scan_omp(**x, init_state=init, return_last_state=True, threads=4)
    ro, rs = oracle.selective_scan(**x, init_state=init, return_last_state=True)
    assert np.array_equal(o, ro) and np.array_equal(s, rs)
    st = {k: (v[:, 0] if k in ("u", "delta", "z", "B", "C") else v) for k, v in x.items()}
    so, ss = oracle.selective_state_update_omp(init, **st, threads=2)
    ro, rs = oracle.selective_state_update(init, **st)
    assert np.array_equal(so, ro) and np.array_equal(ss, rs)


def test_omp_linear_conv_norm_are_bit_identical_to_the_serial_restatement():
    """The blocked product (full 4x64 tiles and ragged edges, bias, silu), the row-parallel conv
    and RMSNorm give the sequential functions' values exactly, as do the reference-shaped Linear
    and the compositions built on each set of primitives."""
    rng = np.random.default_rng(60)
    for R, IN, OUT in ((8, 96, 128), (7, 33, 70), (1, 5, 3), (130, 64, 200)):
        X = rng.standard_normal((R, IN)).astype(F)
        W = rng.standard_normal((OUT, IN)).astype(F)
        b = rng.standard_normal(OUT).astype(F)
        for bias, act in ((None, 0), (b, 0), (b, 1)):
            want = oracle.linear(X, W, bias, act)
            assert np.array_equal(oracle.linear_omp(X, W, bias, act, threads=3), want), (R, IN, OUT, act)
        assert np.array_equal(oracle.r_linear(X, W, b), oracle.linear(X, W, b))
    x = rng.standard_normal((3, 20, 37)).astype(F)
    w = rng.standard_normal((37, 4)).astype(F)
    cb = rng.standard_normal(37).astype(F)
    assert np.array_equal(oracle.conv1d_silu_omp(x, w, cb, threads=3), oracle.conv1d_silu(x, w, cb))
    X = rng.standard_normal((9, 40)).astype(F)
    g = rng.standard_normal(40).astype(F)
    assert np.array_equal(oracle.rmsnorm_omp(X, g, 1e-5, threads=2), oracle.rmsnorm(X, g, 1e-5))
    from tests.util import block_inputs, lm_params
    p = block_inputs(2, 24, 16, 32, 16, 8, 4, seed=61)
    want = oracle.mamba_block(**p, dt_rank=8, bf16=False)
    assert np.array_equal(oracle.mamba_block(**p, dt_rank=8, bf16=False, impl="omp", threads=3), want)
    assert np.array_equal(oracle.mamba_block(**p, dt_rank=8, bf16=False, impl="ref"), want)
    P = lm_params(2, 32, 64, 16, 8, 4, 256, seed=62)
    tok = np.random.default_rng(63).integers(0, 256, (3, 10))
    lg, st = oracle.lm_prefill(tok[:, :9], P, 8, bf16=False)
    lo, so = oracle.lm_prefill(tok[:, :9], P, 8, bf16=False, impl="omp", threads=3)
    assert np.array_equal(lo, lg)
    dl, _ = oracle.lm_decode_step(tok[:, 9], P, st, 8, bf16=False)
    do, _ = oracle.lm_decode_step(tok[:, 9], P, so, 8, bf16=False, impl="omp", threads=2)
    assert np.array_equal(do, dl)


def test_s4d_complex_omp_f32_within_rounding_of_the_f64_checker():
    rng = np.random.default_rng(64)
    Bt, L, Dd, N = 2, 700, 37, 16
    x = rng.standard_normal((Bt, L, Dd)).astype(F)
    prm = dict(dt=np.full(Dd, 0.1, F), a_re=np.full((Dd, N), -0.5, F),
               a_im=np.tile(np.pi * np.arange(N, dtype=F), (Dd, 1)),
               B_re=(rng.standard_normal((Dd, N)) * 0.1).astype(F),
               B_im=(rng.standard_normal((Dd, N)) * 0.1).astype(F),
               C_re=(rng.standard_normal((Dd, N)) * 0.1).astype(F),
               C_im=(rng.standard_normal((Dd, N)) * 0.1).astype(F),
               D=rng.standard_normal(Dd).astype(F))
    ref = oracle.s4d_complex(x, **prm)
    got = oracle.s4d_complex_omp(x, **prm, threads=3)
    assert got.dtype == np.float32 and norm_err(got, ref) < 1e-5
    # a dropped imaginary coupling is far outside that bar
    bad = oracle.s4d_complex_omp(x, **dict(prm, C_im=np.zeros_like(prm["C_im"])), threads=3)
    assert norm_err(bad, ref) > 1e-2


def test_scan_softplus_threshold():
    # delta_raw > 20 passes through unchanged: h = exp(d*A) h + d*u*B with d = delta_raw
    L = 3
    f = lambda v, shape: np.full(shape, v, F)
    out = oracle.selective_scan(f(1.0, (1, L, 1)), f(25.0, (1, L, 1)), f(-0.01, (1, 1)),
                                f(1.0, (1, L, 1)), f(1.0, (1, L, 1)))
    out_np = oracle.selective_scan(f(1.0, (1, L, 1)), f(25.0, (1, L, 1)), f(-0.01, (1, 1)),
                                   f(1.0, (1, L, 1)), f(1.0, (1, L, 1)), delta_softplus=False)
    assert np.array_equal(out, out_np)


# ------------------------------------------------------------------ S4D complex

def s4d_params(dim, N, seed):
    rng = np.random.default_rng(seed)
    return dict(
        dt=np.full(dim, 0.1, F),
        a_re=np.full((dim, N), -0.5, F),
        a_im=np.tile((np.pi * np.arange(N)).astype(F), (dim, 1)),
        B_re=rng.standard_normal((dim, N)).astype(F), B_im=rng.standard_normal((dim, N)).astype(F),
        C_re=rng.standard_normal((dim, N)).astype(F), C_im=rng.standard_normal((dim, N)).astype(F),
        D=rng.standard_normal(dim).astype(F),
    )


def test_s4d_impulse_response():
    dim, N, L = 3, 4, 20
    p = s4d_params(dim, N, 0)
    x = np.zeros((1, L, dim), F)
    x[0, 0, :] = 1.0
    y = oracle.s4d_complex(x, **p)
    q = {k: v.astype(np.float64) for k, v in p.items()}
    Ab = np.exp(q["dt"][:, None] * (q["a_re"] + 1j * q["a_im"]))
    Bb = q["dt"][:, None] * (q["B_re"] + 1j * q["B_im"])
    Cc = q["C_re"] + 1j * q["C_im"]
    for t in range(L):
        ref = 2 * np.real((Cc * Ab ** t * Bb).sum(-1)) + (p["D"] if t == 0 else 0)
        assert rel_err(y[0, t], ref) < 1e-6


def test_s4d_constant_input_steady_state():
    dim, N, L = 2, 3, 400
    p = s4d_params(dim, N, 1)
    x = np.ones((1, L, dim), F)
    y = oracle.s4d_complex(x, **p)
    q = {k: v.astype(np.float64) for k, v in p.items()}
    Ab = np.exp(q["dt"][:, None] * (q["a_re"] + 1j * q["a_im"]))
    Bb = q["dt"][:, None] * (q["B_re"] + 1j * q["B_im"])
    Cc = q["C_re"] + 1j * q["C_im"]
    ss = 2 * np.real((Cc * Bb / (1 - Ab)).sum(-1)) + p["D"]
    assert rel_err(y[0, -1], ss) < 1e-6


# ------------------------------------------------------------------ planted mistakes (the checks bite)

# ------------------------------------------------------------------ Mamba block pieces

def test_conv1d_width1_closed_form():
    rng = np.random.default_rng(30)
    x = rng.standard_normal((2, 7, 5)).astype(F)
    w = rng.standard_normal((5, 1)).astype(F)
    b = rng.standard_normal(5).astype(F)
    pre = x.astype(np.float64) * w[:, 0] + b
    assert rel_err(oracle.conv1d_silu(x, w, b), pre / (1 + np.exp(-pre))) < 1e-6


def test_conv1d_impulse_gives_reversed_taps_and_is_causal():
    W, L = 4, 9
    w = np.arange(1, 2 * W + 1, dtype=F).reshape(2, W) * F(0.25)
    x = np.zeros((1, L, 2), F)
    x[0, 3, :] = 1.0
    y = oracle.conv1d_silu(x, w)[0].astype(np.float64)
    sil = lambda v: v / (1 + np.exp(-v))  # noqa: E731
    for d in range(2):
        for t in range(L):
            j = t - 3  # the impulse at time 3 meets tap W-1-j at output t
            expect = w[d, W - 1 - j] if 0 <= j < W else 0.0
            assert abs(y[t, d] - sil(expect)) < 1e-6, (d, t)
    # causality: changing x at t >= 5 leaves outputs before 5 untouched
    x2 = x.copy()
    x2[0, 5:, :] = 7.0
    assert np.array_equal(oracle.conv1d_silu(x2, w)[0, :5], oracle.conv1d_silu(x, w)[0, :5])


def test_conv1d_vs_numpy_convolve():
    rng = np.random.default_rng(31)
    x = rng.standard_normal((3, 20, 6)).astype(F)
    w = rng.standard_normal((6, 4)).astype(F)
    b = rng.standard_normal(6).astype(F)
    assert rel_err(oracle.conv1d_silu(x, w, b), oracle.numpy_conv1d_silu(x, w, b)) < 1e-5


def test_bf16_round_matches_torch():
    import torch
    rng = np.random.default_rng(32)
    a = (rng.standard_normal(4096) * 10.0 ** rng.integers(-20, 20, 4096)).astype(F)
    a[:4] = [0.0, -0.0, np.inf, -np.inf]
    want = torch.from_numpy(a).to(torch.bfloat16).float().numpy()
    assert np.array_equal(oracle.bf16_round(a), want)


def test_mamba_block_vs_numpy_f64():
    from tests.util import block_inputs
    p = block_inputs(2, 24, 16, 32, 16, 8, 4, seed=33)
    y = oracle.mamba_block(**p, dt_rank=8)
    r = oracle.numpy_mamba_block(**p, dt_rank=8)
    assert y.shape == (2, 24, 16)
    # both round the same storage points to bf16; a one-ulp bf16 flip of an intermediate is the
    # largest legitimate difference
    assert rel_err(y, r) < 2e-2


def test_mamba_block_f64_state_and_unrounded_output():
    """The float64 twin's layer options: its decode hand-off equals the f32 restatement's conv
    window exactly (both hold bf16 values) and its scan state to rounding; round_out=False skips
    only the final rounding."""
    from tests.util import block_inputs
    p = block_inputs(2, 24, 16, 32, 16, 8, 4, seed=35)
    y, last, conv = oracle.mamba_block(**p, dt_rank=8, round_out=False, return_state=True)
    y64, last64, conv64 = oracle.numpy_mamba_block(**p, dt_rank=8, round_out=False, return_state=True)
    assert np.array_equal(conv64, conv)
    assert rel_err(last64, last) < 1e-2
    assert norm_err(y64, y) < 1e-2
    assert np.array_equal(oracle.bf16_round(y64.astype(np.float32)),
                          oracle.bf16_round(oracle.numpy_mamba_block(**p, dt_rank=8).astype(np.float32)))


def test_lm_f64_twin_matches_f32_oracle_and_catches_a_dropped_norm():
    """The float64 twins of the byte LM (prefill, decode) agree with the pinned f32 restatement
    to the bf16 storage bar (they share every rounding point); a twin that skips a layer's
    RMSNorm weight does not."""
    from tests.util import lm_params
    P = lm_params(2, 32, 64, 16, 8, 4, 256, seed=45)
    tok = np.random.default_rng(46).integers(0, 256, (3, 12))
    lg, st = oracle.lm_prefill(tok[:, :11], P, 8)
    lg64, st64 = oracle.numpy_lm_prefill(tok[:, :11], P, 8)
    assert norm_err(lg64, lg) < 1e-2
    for (a, b), (c, d) in zip(st, st64):
        assert np.array_equal(b, d) and rel_err(c, a) < 1e-2
    dl, _ = oracle.lm_decode_step(tok[:, 11], P, st, 8)
    dl64, _ = oracle.numpy_lm_decode_step(tok[:, 11], P, st64, 8)
    assert norm_err(dl64, dl) < 1e-2
    full64, _ = oracle.numpy_lm_prefill(tok, P, 8)
    assert norm_err(dl64, full64[:, 11]) < 1e-2
    bad = dict(P, layers=[dict(P["layers"][0], norm_w=np.ones_like(P["layers"][0]["norm_w"])),
                          P["layers"][1]])
    lgb, _ = oracle.numpy_lm_prefill(tok[:, :11], bad, 8)
    assert norm_err(lgb, lg) > 5e-2


def test_s4_ref_omp_is_bit_identical_to_the_serial_restatement():
    M, N, L = 96, 16, 1500
    p = s4_params(M, N, 24)
    x = np.random.default_rng(25).standard_normal((M, L)).astype(F)
    gate = np.random.default_rng(26).standard_normal(M).astype(F)
    assert np.array_equal(oracle.s4_ref_fwd_omp(x, **p, gate=gate, threads=4), oracle.s4_ref_fwd(x, **p, gate=gate))
    assert np.array_equal(oracle.s4_ref_fwd_omp(x, **p, threads=3), oracle.s4_ref_fwd(x, **p))


def test_s4_ref_f64_matches_numpy_and_f32():
    M, N, L = 24, 16, 300
    p = s4_params(M, N, 21, a_real=np.full(N, -0.5), a_imag=np.pi * np.arange(N))
    x = np.random.default_rng(22).standard_normal((M, L)).astype(F)
    gate = np.random.default_rng(23).standard_normal(M).astype(F)
    y64 = oracle.s4_ref_fwd(x, **p, gate=gate, f64=True)
    assert y64.dtype == np.float64
    # the C restatement widens the reference's f32 dt = 0.1f; give numpy the same value
    r = oracle.numpy_s4_ref(x, **p, gate=gate, dt=float(np.float32(0.1)))
    assert rel_err(y64, r) < 1e-12
    assert rel_err(oracle.s4_ref_fwd(x, **p, gate=gate), y64) < 1e-4


def test_conv1d_step_equals_last_conv_output():
    rng = np.random.default_rng(40)
    x = rng.standard_normal((2, 9, 12)).astype(F)
    w = rng.standard_normal((12, 4)).astype(F)
    b = rng.standard_normal(12).astype(F)
    full = oracle.conv1d_silu(x, w, b)
    state = np.zeros((2, 3, 12), F)
    for t in range(9):
        y, state = oracle.conv1d_step(x[:, t], w, b, state)
        assert np.array_equal(y, full[:, t]), t


def test_lm_decode_after_prefill_equals_longer_prefill():
    from tests.util import lm_params
    P = lm_params(2, 32, 64, 16, 8, 4, 256, seed=41)
    tok = np.random.default_rng(42).integers(0, 256, (3, 11))
    full, _ = oracle.lm_prefill(tok, P, 8)
    pre, st = oracle.lm_prefill(tok[:, :9], P, 8)
    assert np.array_equal(pre, full[:, :9])
    d1, st = oracle.lm_decode_step(tok[:, 9], P, st, 8)
    d2, st = oracle.lm_decode_step(tok[:, 10], P, st, 8)
    assert rel_err(d1, full[:, 9]) < 1e-5 and rel_err(d2, full[:, 10]) < 1e-5


def test_lm_zero_layers_is_head_of_embedding():
    from tests.util import lm_params
    P = lm_params(0, 32, 64, 16, 8, 4, 256, seed=43)
    tok = np.array([[0, 255, 7]])
    lg, _ = oracle.lm_prefill(tok, P, 8)
    xn = oracle.bf16_round(P["embed"][tok[0]] / np.sqrt((P["embed"][tok[0]] ** 2).mean(-1, keepdims=True) + 1e-5)
                           * P["norm_f"])
    ref = xn.astype(np.float64) @ P["w_head"].astype(np.float64).T
    assert rel_err(lg[0], ref) < 1e-2  # one bf16 flip of the normalised input at most


def test_rmsnorm_random_eps_is_below_resolution():
    # the reference draws eps' ~ U[eps, eps + 1e-8) per row (nn/src/lib.rs:262); on rows with
    # mean square >= 1e-2 the jitter is below f32 resolution of ms + eps, so a fixed eps agrees
    rng = np.random.default_rng(44)
    x = rng.standard_normal((64, 512)).astype(F)
    w = rng.standard_normal(512).astype(F)
    y0 = oracle.rmsnorm(x, w, 1e-5)
    for _ in range(3):
        ej = np.float32(1e-5 + rng.uniform(0, 1e-8))
        assert rel_err(oracle.rmsnorm(x, w, ej), y0) < 1e-6


# ------------------------------------------------------------------ tensor primitives

def test_unary_special_values_and_f64():
    z = np.zeros(3, F)
    assert np.all(oracle.unary("exp", z) == 1) and np.all(oracle.unary("cos", z) == 1)
    assert np.all(oracle.unary("sin", z) == 0) and np.all(oracle.unary("log", np.ones(3, F)) == 0)
    sq = np.array([0, 1, 4, 9, 1 << 20], F)
    assert np.array_equal(oracle.unary("sqrt", sq * sq), sq)
    x = np.random.default_rng(4).standard_normal(10000).astype(F) * F(3)
    for op, f in (("exp", np.exp), ("sin", np.sin), ("cos", np.cos)):
        r = f(x.astype(np.float64))
        g = oracle.unary(op, x).astype(np.float64)
        ulp = np.spacing(np.abs(r).astype(F)).astype(np.float64)
        assert np.all(np.abs(g - r) <= ulp), op          # within one f32 ulp of the exact value
    xd = x.astype(np.float64)
    assert rel_err(oracle.unary("silu", x), xd / (1 + np.exp(-xd))) < 1e-6
    assert rel_err(oracle.unary("sigmoid", x), 1 / (1 + np.exp(-xd))) < 1e-6
    assert np.array_equal(oracle.unary("mul_scalar", x, 0.5), x * F(0.5))
    assert np.array_equal(oracle.unary("neg", x), -x)


def test_mean_axis_closed_forms_and_order():
    # constant rows and small integers: exact in any order
    assert np.all(oracle.mean_axis(np.full((3, 24), 2.5, F), 1) == F(2.5))
    ints = np.arange(40, dtype=F).reshape(4, 10)
    assert np.array_equal(oracle.mean_axis(ints, 1), ints.sum(1) / F(10))
    assert np.array_equal(oracle.mean_axis(ints, 0), ints.sum(0) / F(4))
    # summation order, derived by hand from ndarray's fold: row [1e8, 1, 1, 1, -1e8, 1, 1, 1, 0]
    # folds to p0 + p4 = 0, then + 2 + 2 + 2 = 6 (sequentially 1e8 absorbs the first three ones: 3)
    row = np.array([1e8, 1, 1, 1, -1e8, 1, 1, 1, 0], F)
    assert oracle.mean_axis(row[None, :], 1)[0] == F(6) / F(9)
    assert oracle.mean_axis(row[:, None], 0)[0] == F(3) / F(9)
    x = np.random.default_rng(2).standard_normal((5, 37)).astype(F)
    assert rel_err(oracle.mean_axis(x, 1), x.astype(np.float64).mean(1)) < 1e-5


def test_rmsnorm_ref_matches_rmsnorm_to_rounding():
    x = np.random.default_rng(3).standard_normal((8, 64)).astype(F)
    w = np.random.default_rng(4).standard_normal(64).astype(F)
    assert rel_err(oracle.rmsnorm_ref(x, w, 1e-5), oracle.rmsnorm(x, w, 1e-5)) < 1e-6


def test_broadcast_to_restatement():
    rng = np.random.default_rng(6)
    for src, dst in [((5,), (3, 5)), ((4, 5), (3, 4, 5)), ((1, 5), (2, 3, 5)), ((5,), (2, 3, 5)),
                     ((2, 3, 1), (2, 3, 7)), ((3,), (2, 2, 2, 3)), ((1, 2, 1, 3), (2, 2, 4, 3))]:
        x = rng.standard_normal(src).astype(F)
        assert np.array_equal(oracle.broadcast_to(x, dst), np.broadcast_to(x, dst)), (src, dst)
    # (1,2) with len == rows == 1: the repeat-columns branch (lib.rs:1405-1419)
    assert np.array_equal(oracle.broadcast_to(np.array([7], F), (1, 4)), np.full((1, 4), 7, F))
    # generic index map with a rank gap and a >1 source rank (lib.rs:531-546): target dim j reads
    # stride self_strides[j] or 1 past the source rank; for [2, 3] -> [1, 1, 2, 3] both source
    # dims get stride 1, so out[..., r, c] = src_flat[r + c]
    x = np.arange(6, dtype=F).reshape(2, 3)
    assert np.array_equal(oracle.broadcast_to(x, (1, 1, 2, 3)).reshape(2, 3),
                          np.array([[0, 1, 2], [1, 2, 3]], F))
    with pytest.raises(ValueError):
        oracle.broadcast_to(np.ones(4, F), (3, 5))
    with pytest.raises(ValueError):
        oracle.broadcast_to(np.ones(1, F), (3, 5))   # size-1 vector, R and C > 1


def test_stack_restatement():
    a, b = np.arange(3, dtype=F), np.arange(3, 6, dtype=F)
    data, field = oracle.stack([a, b], 1)
    assert field == [3, 2] and np.array_equal(data.reshape(-1), np.arange(6, dtype=F))
    xs = [np.random.default_rng(k).standard_normal((2, 3, 2, 2)).astype(F) for k in range(3)]
    data, field = oracle.stack(xs, 2)
    assert field == [2, 3, 3, 2, 2] and np.array_equal(data, np.stack(xs, 2))


def test_planted_mistakes_are_caught():
    x = inputs(1, 50, 4, 16, 6)
    good = oracle.selective_scan(**x)
    ref, _ = oracle.numpy_selective_scan(**x)
    assert rel_err(good, ref) < 1e-4
    # dropped D term
    assert rel_err(oracle.selective_scan(**{**x, "D": None}), ref) > 1e-2
    # B and C transposed
    assert rel_err(oracle.selective_scan(**{**x, "B": x["C"], "C": x["B"]}), ref) > 1e-2
    # sign of A flipped (on a short sequence so it stays finite)
    short = {n: (v[:, :8] if n in ("u", "delta", "B", "C", "z") else v) for n, v in x.items()}
    ref_s, _ = oracle.numpy_selective_scan(**short)
    assert rel_err(oracle.selective_scan(**{**short, "A": -short["A"]}), ref_s) > 1e-3
    # S4: wrong decay (cos replaced by 1) is caught by the closed form
    M, N, L = 4, 4, 10
    p = s4_params(M, N, 12, a_real=np.full(N, -0.5), a_imag=np.pi * np.arange(N))
    x1 = np.random.default_rng(13).standard_normal((M, L)).astype(F)
    wrong = dict(p, a_imag=np.zeros(N, F))
    assert rel_err(oracle.s4_ref_fwd(x1, **wrong), oracle.numpy_s4_ref(x1, **p)) > 1e-2
    # conv taps applied in forward instead of reversed order
    xc = np.random.default_rng(14).standard_normal((1, 12, 3)).astype(F)
    wc = np.random.default_rng(15).standard_normal((3, 4)).astype(F)
    assert rel_err(oracle.conv1d_silu(xc, wc[:, ::-1]), oracle.numpy_conv1d_silu(xc, wc)) > 1e-2
    # block: x and z halves of in_proj swapped
    from tests.util import block_inputs
    pb = block_inputs(1, 16, 16, 32, 16, 8, 4, seed=16)
    rb = oracle.numpy_mamba_block(**pb, dt_rank=8)
    swapped = dict(pb, w_in=np.concatenate([pb["w_in"][32:], pb["w_in"][:32]]))
    assert rel_err(oracle.mamba_block(**swapped, dt_rank=8), rb) > 1e-1


def test_reference_execution_shape_restatement_is_bit_identical():
    """The (R) CPU-baseline restatement (allocation per op, copied slices, stack) computes the
    same f32 operations in the same order as the pinned oracle: equal bit for bit."""
    rng = np.random.default_rng(41)
    M, N, L = 24, 16, 37
    x = rng.standard_normal((M, L)).astype(F)
    ar = np.full(N, -0.5, F)
    ai = (np.pi * np.arange(N)).astype(F)
    B = (rng.standard_normal((N, M)) * 0.1).astype(F)
    C = (rng.standard_normal((M, N)) * 0.1).astype(F)
    D = rng.standard_normal(M).astype(F)
    assert np.array_equal(oracle.r_s4_forward_ssm(x, ar, ai, B, C, D), oracle.s4_ref_fwd(x, ar, ai, B, C, D))
    X = rng.uniform(-1, 1, (100, 64)).astype(F)
    Wg = (rng.standard_normal((128, 64)) * np.sqrt(2 / 64)).astype(F)
    Wo = (rng.standard_normal((64, 128)) * np.sqrt(2 / 128)).astype(F)
    bg = rng.standard_normal(128).astype(F) * np.float32(0.1)
    bo = rng.standard_normal(64).astype(F) * np.float32(0.1)
    assert np.array_equal(oracle.r_mamba_mlp(X, Wg, bg, Wo, bo), oracle.mamba_mlp(X, Wg, bg, Wo, bo))


def test_componentwise_bar_separates_rounding_from_mistakes():
    """The componentwise metric the block and LM GPU tests use: the f32 restatement sits under one
    bf16 ulp of the output product's term magnitudes from its float64 twin, while a block that
    drops the D skip (about 180 ulps here), swaps the x and z halves of in_proj (about 940) or
    drops dt_bias (about 700), or a head with a mis-scaled final norm weight, lands far outside
    CW_ULPS."""
    from tests.util import CW_ULPS, block_inputs, cw_ulps, lm_params
    p = block_inputs(2, 37, 64, 256, 16, 32, 4, seed=2037)
    ref = oracle.mamba_block(**p, dt_rank=32)
    ref64, terms = oracle.numpy_mamba_block(**p, dt_rank=32, return_terms=True)
    assert cw_ulps(ref, ref64, terms) <= 1.0
    di = p["w_in"].shape[0] // 2
    for bad_p in (dict(p, D=np.zeros_like(p["D"])),
                  dict(p, w_in=np.concatenate([p["w_in"][di:], p["w_in"][:di]], 0)),
                  dict(p, dt_bias=np.zeros_like(p["dt_bias"]))):
        bad = oracle.mamba_block(**bad_p, dt_rank=32)
        assert cw_ulps(bad, ref64, terms) > 4 * CW_ULPS
    P = lm_params(2, 32, 64, 16, 8, 4, 256, seed=47)
    tok = np.random.default_rng(48).integers(0, 256, (2, 9))
    lg, _ = oracle.lm_prefill(tok, P, 8)
    lg64, _, lterms = oracle.numpy_lm_prefill(tok, P, 8, return_terms=True)
    assert cw_ulps(lg, lg64, lterms) <= 1.0
    bad = dict(P, norm_f=np.asarray(P["norm_f"]) * 1.5)
    lgb, _ = oracle.lm_prefill(tok, bad, 8)
    assert cw_ulps(lgb, lg64, lterms) > 4 * CW_ULPS
