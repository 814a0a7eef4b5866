"""Parity of the HIP selective scan (hx_selective_scan_fwd / hx_selective_state_update, called
through the C ABI) against the pinned CPU oracle on identical seeded inputs.

Bars: fp32 storage max rel err <= 1e-4; bf16 storage <= 2e-2 (metric in tests/util.py). Sizes
cover ragged edges (seqlen not a multiple of the 16-step chunk, dim not a multiple of the
64-channel tile), every kernel variant, optional operands, state hand-off, decode, and the
full BASELINE config-2 shape.
"""
import numpy as np
import pytest
import torch

import oracle
from helixml_amd import ssm
from helixml_amd._ffi import InvalidInput, UnsupportedOperation
from tests.util import TOL_BF16, TOL_F32, bf16_round, norm_err, rel_err, scan_inputs

pytestmark = pytest.mark.gpu

# -1 generic, 8 fast, 40 wave-complete, 42 its per-wave-staged form, 44 warp-specialised,
# 46 its split-state form (fp32)
VARIANTS = [-1, 8, 40, 42, 44, 46]


def to_dev(x, dev, dtype=torch.float32):
    return None if x is None else torch.from_numpy(np.ascontiguousarray(x)).to(dev).to(dtype)


def run_gpu(x, dev, dtype=torch.float32, softplus=True, init_state=None, last=False):
    st = dtype
    args = dict(
        u=to_dev(x["u"], dev, st), delta=to_dev(x["delta"], dev, st), A=to_dev(x["A"], dev),
        B=to_dev(x["B"], dev, st), C=to_dev(x["C"], dev, st), D=to_dev(x["D"], dev),
        z=to_dev(x["z"], dev, st), dt_bias=to_dev(x["dt_bias"], dev),
        init_state=to_dev(init_state, dev), delta_softplus=softplus, return_last_state=last)
    r = ssm.selective_scan_fwd(**args)
    torch.cuda.synchronize()
    if last:
        return r[0].float().cpu().numpy(), r[1].cpu().numpy()
    return r.float().cpu().numpy()


@pytest.fixture(autouse=True)
def _reset_variant(dev):
    yield
    ssm.set_scan_variant(0)


SHAPES = [
    (1, 1, 1, 16), (1, 16, 64, 16), (2, 37, 5, 16), (1, 100, 128, 16), (2, 257, 130, 16),
    (3, 48, 192, 16), (1, 64, 64, 4), (1, 50, 33, 7), (2, 33, 70, 32), (1, 20, 10, 64),
]


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("variant", VARIANTS)
def test_scan_matches_oracle(dev, shape, variant):
    bt, L, dim, N = shape
    ssm.set_scan_variant(variant)
    x = scan_inputs(bt, L, dim, N, seed=hash(shape) % 1000, with_bias=True)
    print(f"case variant={variant} shape={shape}", flush=True)
    g = run_gpu(x, dev)
    r = oracle.selective_scan(**x)
    assert rel_err(g, r) <= TOL_F32


@pytest.mark.parametrize("with_z", [True, False])
@pytest.mark.parametrize("with_D", [True, False])
@pytest.mark.parametrize("softplus", [True, False])
@pytest.mark.parametrize("variant", VARIANTS)
def test_scan_optional_operands(dev, with_z, with_D, softplus, variant):
    ssm.set_scan_variant(variant)
    x = scan_inputs(2, 70, 96, 16, seed=7, with_z=with_z, with_D=with_D)
    if not softplus:
        x["delta"] = np.abs(x["delta"]) * np.float32(0.01)  # positive step sizes
    g = run_gpu(x, dev, softplus=softplus)
    r = oracle.selective_scan(**x, delta_softplus=softplus)
    assert rel_err(g, r) <= TOL_F32


@pytest.mark.parametrize("variant", [0, 42, 44, 46, -1])
def test_scan_softplus_all_regimes(dev, variant):
    """delta spread over softplus's regimes: e^x far below f32 resolution of 1 + e^x (x < -17,
    where softplus(x) = e^x), the log1p range, and past the x > 20 cut-over."""
    ssm.set_scan_variant(variant)
    x = scan_inputs(2, 130, 96, 16, seed=21, with_bias=True)
    rng = np.random.default_rng(22)
    x["delta"] = (rng.standard_normal(x["delta"].shape) * 9.0).astype(np.float32)
    x["delta"][:, ::7] = np.float32(-30.0)
    x["delta"][:, 3::11] = np.float32(25.0)
    x["A"] = (x["A"] * np.float32(0.05)).astype(np.float32)  # keep exp(dt*A) away from 0 at dt ~ 25
    g = run_gpu(x, dev)
    assert rel_err(g, oracle.selective_scan(**x)) <= TOL_F32


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_scan_warp_specialised_matches_wave_kernel_bitwise(dev, dtype):
    """The warp-specialised kernel (44) keeps scan_wave3_kernel's (42) operation order, so the
    automatic choice between them never changes a result bit; ragged L and dim included."""
    x = scan_inputs(3, 203, 100, 16, seed=23, with_bias=True)
    init = (np.random.default_rng(24).standard_normal((3, 100, 16)) * 0.5).astype(np.float32)
    outs = {}
    for v in (42, 44):
        ssm.set_scan_variant(v)
        outs[v] = run_gpu(x, dev, dtype=dtype, init_state=init, last=True)
    assert np.array_equal(outs[44][0], outs[42][0])
    assert np.array_equal(outs[44][1], outs[42][1])


def test_scan_general_A(dev):
    x = scan_inputs(2, 300, 130, 16, seed=8, s4d_real_A=False, with_bias=True)
    g = run_gpu(x, dev)
    assert rel_err(g, oracle.selective_scan(**x)) <= TOL_F32


@pytest.mark.parametrize("variant", VARIANTS)
def test_scan_state_handoff(dev, variant):
    ssm.set_scan_variant(variant)
    x = scan_inputs(2, 90, 80, 16, seed=9)
    r, rlast = oracle.selective_scan(**x, return_last_state=True)
    g, glast = run_gpu(x, dev, last=True)
    assert rel_err(g, r) <= TOL_F32
    assert rel_err(glast, rlast) <= TOL_F32
    # split at k: second half seeded with the first half's final state
    k = 41
    seq = ("u", "delta", "B", "C", "z")
    first = {n: (v[:, :k].copy() if n in seq else v) for n, v in x.items()}
    second = {n: (v[:, k:].copy() if n in seq else v) for n, v in x.items()}
    g1, s1 = run_gpu(first, dev, last=True)
    g2, s2 = run_gpu(second, dev, init_state=s1, last=True)
    assert rel_err(np.concatenate([g1, g2], 1), r) <= TOL_F32
    assert rel_err(s2, rlast) <= TOL_F32


def test_scan_zero_length_returns_initial_state(dev):
    x = scan_inputs(2, 0, 8, 16, seed=10)
    init = np.random.default_rng(0).standard_normal((2, 8, 16)).astype(np.float32)
    g, s = run_gpu(x, dev, init_state=init, last=True)
    assert g.shape == (2, 0, 8)
    assert np.array_equal(s, init)


def test_scan_zero_length_without_initial_state_writes_zeros(dev):
    """No initial state: the final state is zero, written by a fill kernel (the output starts as
    NaN, so a skipped write shows), through the plain and the no-allocation entry points."""
    from helixml_amd import _ffi
    x = {k: to_dev(v, dev) for k, v in scan_inputs(2, 0, 8, 16, seed=12).items()}
    out = torch.empty((2, 0, 8), device=dev)
    for entry in ("hx_selective_scan_fwd", "hx_selective_scan_fwd_noalloc"):
        last = torch.full((2, 8, 16), float("nan"), device=dev)
        args = [2, 0, 8, 16, _ffi.HX_F32, 1] + [x[k].data_ptr() if x[k] is not None else None
                                                for k in ("u", "delta", "A", "B", "C", "D", "z",
                                                          "dt_bias")]
        _ffi.call(entry, *args, out.data_ptr(), None, last.data_ptr(),
                  torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        assert torch.equal(last, torch.zeros_like(last)), entry


@pytest.mark.parametrize("variant", VARIANTS)
@pytest.mark.parametrize("shape", [(2, 37, 70, 16), (1, 300, 256, 16)], ids=str)
def test_scan_bf16_storage(dev, variant, shape):
    ssm.set_scan_variant(variant)
    x = scan_inputs(*shape, seed=11)
    xr = {k: (bf16_round(v) if (v is not None and k not in ("A", "D", "dt_bias")) else v)
          for k, v in x.items()}
    g = run_gpu(x, dev, dtype=torch.bfloat16)
    r = oracle.selective_scan(**xr)
    assert rel_err(g, r) <= TOL_BF16


def test_decode_matches_prefill(dev):
    x = scan_inputs(3, 24, 40, 16, seed=12, with_bias=True)
    r, rlast = oracle.selective_scan(**x, return_last_state=True)
    state = torch.zeros((3, 40, 16), device=dev)
    A, D, bias = to_dev(x["A"], dev), to_dev(x["D"], dev), to_dev(x["dt_bias"], dev)
    outs = []
    for t in range(24):
        o = ssm.selective_state_update(state, to_dev(x["u"][:, t], dev), to_dev(x["delta"][:, t], dev), A,
                                       to_dev(x["B"][:, t], dev), to_dev(x["C"][:, t], dev), D,
                                       to_dev(x["z"][:, t], dev), bias)
        outs.append(o.cpu().numpy())
    assert rel_err(np.stack(outs, 1), r) <= TOL_F32
    assert rel_err(state.cpu().numpy(), rlast) <= TOL_F32


def test_decode_after_prefill_handoff(dev):
    x = scan_inputs(4, 33, 64, 16, seed=13)
    r = oracle.selective_scan(**x)
    pre = {n: (v[:, :32].copy() if n in ("u", "delta", "B", "C", "z") else v) for n, v in x.items()}
    g, s = run_gpu(pre, dev, last=True)
    state = to_dev(s, dev)
    o = ssm.selective_state_update(state, to_dev(x["u"][:, 32], dev), to_dev(x["delta"][:, 32], dev),
                                   to_dev(x["A"], dev), to_dev(x["B"][:, 32], dev), to_dev(x["C"][:, 32], dev),
                                   to_dev(x["D"], dev), to_dev(x["z"][:, 32], dev))
    assert rel_err(np.concatenate([g, o.cpu().numpy()[:, None]], 1), r) <= TOL_F32


def test_shape_errors_raise_reference_variants(dev):
    from helixml_amd import DTypeMismatch, ShapeMismatch
    x = scan_inputs(1, 8, 8, 16, seed=14)
    u = to_dev(x["u"], dev)
    with pytest.raises(ShapeMismatch):
        ssm.selective_scan_fwd(u, to_dev(x["delta"][:, :4], dev), to_dev(x["A"], dev),
                               to_dev(x["B"], dev), to_dev(x["C"], dev))
    with pytest.raises(DTypeMismatch):
        ssm.selective_scan_fwd(u, to_dev(x["delta"], dev), to_dev(x["A"], dev).double(),
                               to_dev(x["B"], dev), to_dev(x["C"], dev))


@pytest.mark.parametrize("variant", [0, 40, 42, 44, 46])
def test_baseline_config2_full_size(dev, variant):
    """BASELINE config 2 (batch 8, L 2048, d_inner 1536, d_state 16, fp32) end to end against the
    (multi-threaded, arithmetic-identical) CPU oracle."""
    ssm.set_scan_variant(variant)
    x = scan_inputs(8, 2048, 1536, 16, seed=0xC2)
    try:
        g = run_gpu(x, dev)
    finally:
        ssm.set_scan_variant(0)
    r = oracle.selective_scan_omp(**x)
    err = rel_err(g, r)
    print(f"config2 rel err {err:.3e}")
    assert err <= TOL_F32


@pytest.fixture
def _reset_segments(dev):
    yield
    ssm.set_scan_segments(0)
    ssm.set_scan_variant(0)


@pytest.mark.parametrize("variant", [40, 42])
@pytest.mark.parametrize("nseg", [2, 3, 7])
@pytest.mark.parametrize("shape", [(2, 300, 128, 16), (1, 1000, 64, 16), (1, 77, 192, 16)], ids=str)
def test_scan_segmented_long_sequence_path(dev, _reset_segments, nseg, shape, variant):
    """Time-segmented path (segment end states from zero, carry chain, rescan from entry
    states) against the sequential oracle, with an initial state and the final state checked.

    The final state is compared with the float64 restatement: on (1, 77, 192) the f32 oracle's
    own final state is 1.16e-4 away from it (a component at 1.2e-3 of the largest, 8e-8 off in
    absolute terms), so the bar is the tolerance or 1.5x the f32 oracle's own error, whichever
    is larger."""
    ssm.set_scan_segments(nseg)
    ssm.set_scan_variant(variant)
    x = scan_inputs(*shape, seed=nseg * 11 + shape[1], with_bias=True)
    init = (np.random.default_rng(nseg).standard_normal((shape[0], shape[2], 16)) * 0.5).astype(np.float32)
    r, rlast = oracle.selective_scan(**x, init_state=init, return_last_state=True)
    _, rlast64 = oracle.numpy_selective_scan(**x, init_state=init)
    g, glast = run_gpu(x, dev, init_state=init, last=True)
    assert rel_err(g, r) <= TOL_F32
    assert rel_err(glast, rlast64) <= max(TOL_F32, 1.5 * rel_err(rlast, rlast64))


@pytest.mark.parametrize("zero_a", [False, True])
def test_scan_segmented_decay_window(dev, _reset_segments, zero_a):
    """Segments long enough that the end-state pass starts late: delta_raw ~ N(0, 0.5) (dt about
    0.7) and A = -(n+1), so the decay to a 2048-step segment's end falls below 2^-32 within ~32
    steps and the end states come from that window alone (the carry takes no decay from such a
    segment). With one state's A = 0 in one channel no window applies to that channel's wave;
    that state then sums 8192 undamped terms, whose f32 rounding (in either summation order)
    exceeds the tolerance, so outputs and final state are held to the float64 restatement at the
    tolerance or 1.5x the sequential f32 oracle's own error, whichever is larger."""
    ssm.set_scan_segments(4)
    ssm.set_scan_variant(42)
    x = scan_inputs(1, 8192, 64, 16, seed=0x5E6, with_bias=True)
    x["delta"] = (x["delta"] + np.float32(4.0)).astype(np.float32)
    if zero_a:
        x["A"][5, 3] = 0.0
    print(f"case decay window zero_a={zero_a}", flush=True)
    r, rlast = oracle.selective_scan(**x, return_last_state=True)
    r64, rlast64 = oracle.numpy_selective_scan(**x)
    g, glast = run_gpu(x, dev, last=True)
    print(f"out: gpu {rel_err(g, r64):.3e} f32 oracle {rel_err(r, r64):.3e} vs float64; "
          f"state: gpu {rel_err(glast, rlast64):.3e} f32 oracle {rel_err(rlast, rlast64):.3e}")
    assert rel_err(g, r64) <= max(TOL_F32, 1.5 * rel_err(r, r64))
    assert rel_err(glast, rlast64) <= max(TOL_F32, 1.5 * rel_err(rlast, rlast64))


@pytest.mark.parametrize("variant", [0, 40, 42])
def test_baseline_config4_scan_full_size(dev, variant):
    """BASELINE config 4 scan (batch 1, L 65536, d_inner 2048, d_state 16, fp32): the automatic
    segmented path against the (multi-threaded, arithmetic-identical) CPU oracle."""
    ssm.set_scan_variant(variant)
    x = scan_inputs(1, 65536, 2048, 16, seed=0xC4)
    try:
        g = run_gpu(x, dev)
    finally:
        ssm.set_scan_variant(0)
    r = oracle.selective_scan_omp(**x)
    err = rel_err(g, r)
    print(f"config4 rel err {err:.3e}")
    assert err <= TOL_F32


@pytest.mark.parametrize("variant", [0, 44, 46])
def test_warp_specialised_partial_group_large_offsets(dev, variant):
    """dim % 48 != 0 with a batch row past 2^31 bytes (1 x 30000 x 20000 fp32,
    2.4 GB per operand): the lanes of the last block's channels past dim must not write anywhere.
    Their 32-bit store offsets start past the row's end; advancing them by whole chunks used to
    wrap below it and overwrite channel 18176 (2^32 mod the row size) at early steps. Channels are
    independent, so the oracle runs on the touched channels only, over the whole sequence. Run
    for every warp-specialised kernel and the automatic choice."""
    ssm.set_scan_variant(variant)
    bt, L, dim, N = 1, 30000, 20000, 16
    g = torch.Generator(device=dev).manual_seed(0x5753)
    u = torch.randn((bt, L, dim), generator=g, device=dev)
    delta = torch.randn((bt, L, dim), generator=g, device=dev) * 0.5 - 4.0
    z = torch.randn((bt, L, dim), generator=g, device=dev)
    B = torch.randn((bt, L, N), generator=g, device=dev)
    C = torch.randn((bt, L, N), generator=g, device=dev)
    A = -torch.arange(1, N + 1, device=dev, dtype=torch.float32).repeat(dim, 1).contiguous()
    D = torch.randn((dim,), generator=g, device=dev)
    print(f"case 1x30000x20000 fp32 variant {variant}", flush=True)
    out = ssm.selective_scan_fwd(u, delta, A, B, C, D, z)
    torch.cuda.synchronize()
    chans = [0, 18176, dim - 32, dim - 1]
    cut = lambda t: np.ascontiguousarray(t[:, :, chans].cpu().numpy())  # noqa: E731
    x = dict(u=cut(u), delta=cut(delta), z=cut(z), B=B.cpu().numpy(), C=C.cpu().numpy(),
             A=A[chans].cpu().numpy(), D=D[chans].cpu().numpy(), dt_bias=None)
    del u, delta, z
    r = oracle.selective_scan(**x)
    got = out[:, :, chans].cpu().numpy()
    assert rel_err(got, r) <= TOL_F32


@pytest.mark.parametrize("bt,L,dim,r", [(2, 37, 256, 32), (1, 130, 128, 64), (3, 50, 192, 96),
                                        (1, 33, 256, 128), (2, 1000, 64, 32)])
def test_scan_dtproj_matches_separate_steps(dev, bt, L, dim, r):
    """hx_selective_scan_dtproj_fwd against the block's two separate steps, dt = gemm_bf16(dt_lo,
    w_dt) then the wave kernel (variant 42, whose arithmetic the fused kernel shares): the two
    products sum K in different orders, so a dt value within an fp32 rounding of a bf16 midpoint
    can round the other way and change its channel from that step on. Channels without such a
    flip are bit-identical (most of them), the others agree to the bf16 bar; the fused result is
    held to the oracle with dt rounded as the separate product stores it."""
    g = torch.Generator(device=dev)
    g.manual_seed(bt * 7919 + L * 31 + dim + r)
    bf = torch.bfloat16
    rnd = lambda *s: torch.randn(*s, device=dev, generator=g)  # noqa: E731
    u, z = rnd(bt, L, dim).to(bf), rnd(bt, L, dim).to(bf)
    dt_lo = (rnd(bt, L, r) * 0.5).to(bf)
    w_dt = (rnd(dim, r) / r ** 0.5).to(bf)
    A = -torch.arange(1, 17, device=dev, dtype=torch.float32).repeat(dim, 1).contiguous()
    B, C = rnd(bt, L, 16).to(bf), rnd(bt, L, 16).to(bf)
    D = rnd(dim)
    dt_bias = rnd(dim) * 0.5 - 4.0
    fused, last_f = ssm.selective_scan_dtproj_fwd(u, dt_lo, w_dt, A, B, C, D, z, dt_bias,
                                                  return_last_state=True)
    dt = ssm.gemm_bf16(dt_lo.view(bt * L, r), w_dt).view(bt, L, dim)
    try:
        ssm.set_scan_variant(42)
        sep, last_s = ssm.selective_scan_fwd(u, dt, A, B, C, D, z, dt_bias, return_last_state=True)
    finally:
        ssm.set_scan_variant(0)
    torch.cuda.synchronize()
    same = (fused == sep).all(dim=1)  # [bt, dim]: a channel's whole output
    frac = same.float().mean().item()
    print(f"channels bit-identical to the separate steps: {frac:.3f}", flush=True)
    assert frac >= (0.5 if L >= 1000 else 0.8), frac
    assert torch.equal(last_f[same], last_s[same])
    f, s = fused.float().cpu().numpy(), sep.float().cpu().numpy()
    e_sep = norm_err(f, s)
    x = {k: v.float().cpu().numpy() for k, v in dict(u=u, A=A, B=B, C=C, D=D, z=z, dt_bias=dt_bias).items()}
    dt_ref = bf16_round(oracle.linear(dt_lo.float().cpu().numpy().reshape(-1, r), w_dt.float().cpu().numpy()))
    ref = oracle.selective_scan(x["u"], dt_ref.reshape(bt, L, dim), x["A"], x["B"], x["C"], x["D"], x["z"],
                                x["dt_bias"], True)
    e_ref = norm_err(f, ref)
    print(f"normwise: vs separate steps {e_sep:.3e}, vs oracle {e_ref:.3e}", flush=True)
    assert e_sep <= 4e-3 and e_ref <= 1e-2, (e_sep, e_ref)


def test_scan_dtproj_errors_and_empty(dev):
    """hx_selective_scan_dtproj_fwd takes dt_rank 32, 64, 96 or 128 and dim % 4 == 0 (else
    UnsupportedOperation, nothing launched), needs every operand but D, dt_bias and last_state
    (else InvalidInput), and with no steps sets the final state to zero."""
    from helixml_amd import _ffi
    bf = torch.bfloat16
    bt, L, dim = 2, 16, 64

    def args(r, d=dim, seq=L):
        t = {"u": torch.zeros(bt, seq, d, device=dev, dtype=bf), "dt_lo": torch.zeros(bt, seq, r, device=dev, dtype=bf),
             "w_dt": torch.zeros(d, r, device=dev, dtype=bf), "A": -torch.ones(d, 16, device=dev),
             "B": torch.zeros(bt, seq, 16, device=dev, dtype=bf), "C": torch.zeros(bt, seq, 16, device=dev, dtype=bf),
             "z": torch.zeros(bt, seq, d, device=dev, dtype=bf), "out": torch.zeros(bt, seq, d, device=dev, dtype=bf)}
        return t

    def call(t, r, d=dim, seq=L, last=None, drop=None):
        p = {k: (None if k == drop else v.data_ptr()) for k, v in t.items()}
        _ffi.call("hx_selective_scan_dtproj_fwd", bt, seq, d, r, p["u"], p["dt_lo"], p["w_dt"], p["A"], p["B"],
                  p["C"], None, p["z"], None, p["out"], None if last is None else last.data_ptr(),
                  torch.cuda.current_stream().cuda_stream)

    for r in (16, 48, 160):
        with pytest.raises(UnsupportedOperation):
            call(args(r), r)
    with pytest.raises(UnsupportedOperation):
        call(args(32, d=66), 32, d=66)
    for k in ("u", "dt_lo", "w_dt", "A", "B", "C", "z", "out"):
        with pytest.raises(InvalidInput):
            call(args(32), 32, drop=k)
    last = torch.full((bt, dim, 16), float("nan"), device=dev)
    call(args(64, seq=0), 64, seq=0, last=last)
    torch.cuda.synchronize()
    assert torch.equal(last, torch.zeros_like(last))
