"""Parity of the HIP S4 kernels (hx_s4_ref_fwd, hx_s4d_complex_fwd) against the CPU oracle."""
import numpy as np
import pytest
import torch

import oracle
from helixml_amd import ssm
from tests.util import TOL_F32, norm_err, rel_err

pytestmark = pytest.mark.gpu
F = np.float32


def dv(x, dev):
    return None if x is None else torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def s4_inputs(M, N, L, seed, a_real=None, a_imag=None, D_zero=False):
    # ssm::S4Block::new distributions (crates/nn/src/ssm.rs:42-83): A_real = 0, A_imag ~ N(0,1),
    # B ~ N(0, 0.1) [N, M], C ~ N(0, 0.1) [M, N], D = 0; overridable for config 4's
    # A_real = -0.5, A_imag = pi*n.
    rng = np.random.default_rng(seed)
    return dict(
        x=rng.standard_normal((M, L), dtype=F),
        a_real=np.zeros(N, F) if a_real is None else a_real.astype(F),
        a_imag=rng.standard_normal(N, dtype=F) if a_imag is None else a_imag.astype(F),
        B=(rng.standard_normal((N, M)) * 0.1).astype(F),
        C=(rng.standard_normal((M, N)) * 0.1).astype(F),
        D=np.zeros(M, F) if D_zero else rng.standard_normal(M, dtype=F),
    )


@pytest.mark.parametrize("M,N,L", [(64, 16, 100), (8, 4, 16), (5, 3, 1), (130, 16, 513),
                                   (256, 16, 1000), (33, 64, 70)])
@pytest.mark.parametrize("gated", [False, True])
def test_s4_ref_matches_oracle(dev, M, N, L, gated):
    p = s4_inputs(M, N, L, seed=M * 1000 + L)
    gate = (np.random.default_rng(1).standard_normal(M) * 0.1).astype(F) if gated else None
    print(f"case s4_ref M={M} N={N} L={L} gated={gated}", flush=True)
    g = ssm.s4_ref_fwd(**{k: dv(v, dev) for k, v in p.items()}, gate=dv(gate, dev))
    torch.cuda.synchronize()
    r = oracle.s4_ref_fwd(**p, gate=gate)
    assert g.shape == (L, M)
    assert rel_err(g.cpu().numpy(), r) <= TOL_F32


def test_s4_ref_config4_decay_long(dev):
    # config-4 decay (A_real=-0.5, A_imag=pi*n) over a long sequence, against the float64 restatement
    M, N, L = 128, 16, 20000
    p = s4_inputs(M, N, L, seed=44, a_real=np.full(N, -0.5), a_imag=np.pi * np.arange(N))
    g = ssm.s4_ref_fwd(**{k: dv(v, dev) for k, v in p.items()}).cpu().numpy()
    r = oracle.s4_ref_fwd(**p)
    assert rel_err(g, r) <= TOL_F32


@pytest.mark.parametrize("bt,L,dim,N", [(1, 100, 64, 16), (2, 333, 70, 16), (1, 50, 9, 5), (1, 20, 3, 64)])
def test_s4d_complex_matches_oracle(dev, bt, L, dim, N):
    rng = np.random.default_rng(bt * 7 + L)
    p = dict(
        dt=np.full(dim, 0.1, F),
        a_re=np.full((dim, N), -0.5, F),
        a_im=np.tile((np.pi * np.arange(N)).astype(F), (dim, 1)),
        B_re=(rng.standard_normal((dim, N)) * 0.1).astype(F), B_im=(rng.standard_normal((dim, N)) * 0.1).astype(F),
        C_re=(rng.standard_normal((dim, N)) * 0.1).astype(F), C_im=(rng.standard_normal((dim, N)) * 0.1).astype(F),
        D=rng.standard_normal(dim).astype(F))
    x = rng.standard_normal((bt, L, dim)).astype(F)
    g = ssm.s4d_complex_fwd(dv(x, dev), **{k: dv(v, dev) for k, v in p.items()})
    torch.cuda.synchronize()
    r = oracle.s4d_complex(x, **p)
    assert rel_err(g.cpu().numpy(), r) <= TOL_F32


@pytest.mark.parametrize("M,N,L", [(64, 16, 100), (130, 16, 700), (33, 64, 70)])
def test_s4_ref_bit_exact(dev, M, N, L):
    """Reference mode reproduces CpuTensor's f32 op order, so it is bit-identical to the oracle,
    including the ill-conditioned default init (A_real = 0, |a| ~ 1)."""
    p = s4_inputs(M, N, L, seed=5 + M)
    gate = (np.random.default_rng(2).standard_normal(M) * 0.1).astype(F)
    g = ssm.s4_ref_fwd(**{k: dv(v, dev) for k, v in p.items()}, gate=dv(gate, dev)).cpu().numpy()
    r = oracle.s4_ref_fwd(**p, gate=gate)
    assert np.array_equal(g, r), f"max abs diff {np.abs(g - r).max()}"


# Each case takes a different route through hx_s4_ref_fwd's kernels: the projection's 16- or
# 4-byte ring loads (L % 4, alignment of x) and its tail chunk (M % 16); the streamed
# recurrence (N a power of two, L*N % 4 == 0; several ring wraps at L*N >> 3 x 4096) or the
# per-lane one; the scalar-operand output kernel (N in {4, 8, 16}, L % 4 == 0) or the LDS one.
@pytest.mark.parametrize("M,N,L,offset", [
    (64, 16, 4096, 0),    # all fast paths, 16 recurrence chunks
    (300, 4, 3000, 0),    # 18 full projection chunks + a 12-row tail, N 4 output kernel
    (37, 8, 1003, 0),     # odd L: 4-byte ring loads, streamed recurrence, LDS output kernel
    (19, 2, 6000, 0),     # N 2: 2048-step recurrence chunks
    (19, 1, 2050, 0),     # N 1, L*N % 4 != 0: per-lane recurrence
    (65, 32, 520, 0),     # 4 state groups, 128-step chunks
    (5, 16, 7, 0),        # fewer rows and steps than one tile
    (64, 16, 4096, 1),    # x not 16-byte aligned: 4-byte ring loads, LDS output kernel
    (48, 12, 900, 0),     # N 12: padded state group, per-lane recurrence
])
def test_s4_ref_bit_exact_paths(dev, M, N, L, offset):
    p = s4_inputs(M, N, L, seed=11 + M + N + L, a_real=np.full(N, -0.01))
    gate = (np.random.default_rng(3).standard_normal(M) * 0.1).astype(F)
    print(f"case s4_ref_paths M={M} N={N} L={L} offset={offset}", flush=True)
    d = {k: dv(v, dev) for k, v in p.items()}
    if offset:
        flat = torch.empty(M * L + offset, device=dev, dtype=torch.float32)
        d["x"] = flat[offset:].view(M, L)
        d["x"].copy_(torch.from_numpy(p["x"]))
        assert d["x"].data_ptr() % 16 != 0
    g = ssm.s4_ref_fwd(**d, gate=dv(gate, dev)).cpu().numpy()
    r = oracle.s4_ref_fwd(**p, gate=gate)
    assert np.array_equal(g, r), f"max abs diff {np.abs(g - r).max()}"


# ------------------------------------------------------------------ time-parallel reference mode

@pytest.mark.parametrize("M,N,L", [(64, 16, 100), (8, 4, 16), (5, 3, 1), (130, 16, 513),
                                   (256, 16, 1000), (40, 16, 4099), (64, 5, 2048)])
@pytest.mark.parametrize("gated", [False, True])
@pytest.mark.parametrize("init", ["decay", "default"])
def test_s4_ref_parallel_matches_oracle(dev, M, N, L, gated, init):
    """init "decay": config 4's A (|a| <= e^-0.05), compared with the f32 oracle at 1e-4.
    init "default": the reference's own init (A_real = 0, so |a| = |cos(0.1 A_imag)| ~ 1 - 1e-5):
    the recurrence is ill-conditioned and the reference's f32 result itself is off the exact
    value by up to ~5e-3 at these lengths (elementwise, near-zero outputs). The parallel path
    rounds differently, so it is held to the fp32 bar normwise against the f32 oracle, and
    elementwise to the same order as the reference's own distance from the float64 restatement
    (twice it: both share the f32 rounding of a and Bd)."""
    if init == "decay":
        p = s4_inputs(M, N, L, seed=M * 31 + L, a_real=np.full(N, -0.5), a_imag=np.pi * np.arange(N))
    else:
        p = s4_inputs(M, N, L, seed=M * 31 + L)
    gate = np.random.default_rng(L).standard_normal(M).astype(F) if gated else None
    g = ssm.s4_ref_fwd(**{k: dv(v, dev) for k, v in p.items()}, gate=dv(gate, dev), parallel=True)
    torch.cuda.synchronize()
    g = g.cpu().numpy()
    r32 = oracle.s4_ref_fwd(**p, gate=gate)
    if init == "decay":
        err = rel_err(g, r32)
        assert err <= TOL_F32, err
    else:
        r64 = oracle.numpy_s4_ref(**p, gate=gate)
        err, ref_err = rel_err(g, r64), rel_err(r32, r64)
        nerr = norm_err(g, r32)
        assert nerr <= TOL_F32, nerr
        assert err <= 2 * max(TOL_F32, ref_err), (err, ref_err)


def test_s4_ref_parallel_rejects_large_dstate(dev):
    from helixml_amd._ffi import UnsupportedOperation
    p = s4_inputs(8, 32, 10, seed=1)
    with pytest.raises(UnsupportedOperation):
        ssm.s4_ref_fwd(**{k: dv(v, dev) for k, v in p.items()}, parallel=True)


def test_s4_ref_parallel_config4_full_size(dev):
    """BASELINE config 4, S4 reference mode: d_model 2048, N 16, L 65536, A_real = -0.5,
    A_imag = pi*n, dt = 0.1, over the whole sequence. At this size the f32 reference's own
    elementwise distance from the exact (float64) result is 1.15e-4 (its 2048-term sequential
    sums), so the parallel path is held to 1e-4 against the float64 restatement, and normwise
    to 1e-6 against the f32 restatement."""
    M, N, L = 2048, 16, 65536
    p = s4_inputs(M, N, L, seed=404, a_real=np.full(N, -0.5), a_imag=np.pi * np.arange(N))
    g = ssm.s4_ref_fwd(**{k: dv(v, dev) for k, v in p.items()}, parallel=True)
    torch.cuda.synchronize()
    g = g.cpu().numpy()
    err64 = rel_err(g, oracle.s4_ref_fwd(**p, f64=True))
    assert err64 <= TOL_F32, err64
    nerr = norm_err(g, oracle.s4_ref_fwd_omp(**p))
    assert nerr <= 1e-6, nerr


def test_s4_ref_exact_config4_full_size(dev):
    """BASELINE config 4, S4 reference mode as the bench's exact leg times it (hx_s4_ref_fwd):
    d_model 2048, N 16, L 65536, A_real = -0.5, A_imag = pi*n, over the whole sequence, bit for
    bit against the f32 restatement (its OpenMP form, bit-identical to the sequential one:
    tests/test_oracle.py)."""
    M, N, L = 2048, 16, 65536
    p = s4_inputs(M, N, L, seed=405, a_real=np.full(N, -0.5), a_imag=np.pi * np.arange(N))
    print("case s4 exact 2048x16x65536", flush=True)
    g = ssm.s4_ref_fwd(**{k: dv(v, dev) for k, v in p.items()})
    torch.cuda.synchronize()
    g = g.cpu().numpy()
    r = oracle.s4_ref_fwd_omp(**p)
    assert np.array_equal(g, r), f"max abs diff {np.abs(g - r).max()}"


# ------------------------------------------------------------------ S4D complex, wave path

def s4d_inputs(bt, L, dim, N, seed):
    rng = np.random.default_rng(seed)
    p = dict(
        dt=np.full(dim, 0.1, F),
        a_re=np.full((dim, N), -0.5, F),
        a_im=np.tile((np.pi * np.arange(N)).astype(F), (dim, 1)),
        B_re=(rng.standard_normal((dim, N)) * 0.1).astype(F), B_im=(rng.standard_normal((dim, N)) * 0.1).astype(F),
        C_re=(rng.standard_normal((dim, N)) * 0.1).astype(F), C_im=(rng.standard_normal((dim, N)) * 0.1).astype(F),
        D=rng.standard_normal(dim).astype(F))
    return rng.standard_normal((bt, L, dim), dtype=F), p


@pytest.mark.parametrize("bt,L,dim,nseg", [(1, 100, 64, 0), (2, 333, 72, 0), (1, 1000, 128, 3),
                                           (3, 517, 16, 7), (1, 4096, 256, 0), (1, 17, 64, 2)])
def test_s4d_wave_path(dev, bt, L, dim, nseg):
    x, p = s4d_inputs(bt, L, dim, 16, seed=L + dim)
    ssm.set_s4d_segments(nseg)
    try:
        g = ssm.s4d_complex_fwd(dv(x, dev), **{k: dv(v, dev) for k, v in p.items()})
        torch.cuda.synchronize()
    finally:
        ssm.set_s4d_segments(0)
    err = rel_err(g.cpu().numpy(), oracle.s4d_complex(x, **p))
    assert err <= TOL_F32, err


@pytest.mark.parametrize("slow_channel", [False, True])
def test_s4d_segment_decay_window(dev, slow_channel):
    """2048-step segments with |Abar| = exp(-0.05): the end-state pass starts ~450 steps before a
    segment's end (decay below 2^-32 from there). With one channel's a_re = -0.1 (|Abar| =
    exp(-0.01): 2^-32 only after ~2220 steps) its block has no window and runs whole segments.
    (Much slower decays are not a fair test at this bar: over thousands of undamped rotations the
    one-ulp difference between device and host sincosf in Abar drifts the phase by ~1e-3.)"""
    x, p = s4d_inputs(1, 8192, 64, 16, seed=77)
    if slow_channel:
        p["a_re"][40, :] = np.float32(-0.1)
    print(f"case s4d window slow_channel={slow_channel}", flush=True)
    ssm.set_s4d_segments(4)
    try:
        g = ssm.s4d_complex_fwd(dv(x, dev), **{k: dv(v, dev) for k, v in p.items()})
        torch.cuda.synchronize()
    finally:
        ssm.set_s4d_segments(0)
    err = rel_err(g.cpu().numpy(), oracle.s4d_complex(x, **p))
    assert err <= TOL_F32, err


def test_s4d_wave_path_equals_thread_path(dev):
    x, p = s4d_inputs(2, 300, 64, 16, seed=9)
    args = (dv(x, dev),)
    kw = {k: dv(v, dev) for k, v in p.items()}
    g1 = ssm.s4d_complex_fwd(*args, **kw)
    ssm.set_s4d_path(1)
    try:
        g2 = ssm.s4d_complex_fwd(*args, **kw)
    finally:
        ssm.set_s4d_path(0)
    err = rel_err(g1.cpu().numpy(), g2.cpu().numpy())
    assert err <= TOL_F32, err


def test_s4d_config4_full_size(dev):
    """BASELINE config 4, S4D complex: batch 1, L 65536, d 2048, N 16 (A = -0.5 + i*pi*n).
    Channels are independent, so the oracle checks the first and last 16 channels and every
    8th channel (256 more, spread over every block and wave of the grid) over the whole sequence
    (every segment boundary and carry), and the whole output is finite."""
    bt, L, dim = 1, 65536, 2048
    x, p = s4d_inputs(bt, L, dim, 16, seed=4)
    g = ssm.s4d_complex_fwd(dv(x, dev), **{k: dv(v, dev) for k, v in p.items()})
    torch.cuda.synchronize()
    assert torch.isfinite(g).all()
    gh = g.cpu().numpy()
    for sl in (slice(0, 16), slice(dim - 16, dim), slice(3, dim, 8)):
        ps = {k: (np.ascontiguousarray(v[sl]) if v.ndim >= 1 else v) for k, v in p.items()}
        r = oracle.s4d_complex(np.ascontiguousarray(x[:, :, sl]), **ps)
        err = rel_err(gh[:, :, sl], r)
        assert err <= TOL_F32, (sl, err)
