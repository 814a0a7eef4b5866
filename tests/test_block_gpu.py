"""Mamba block forward on the GPU (hx_conv1d_silu, hx_mamba_block_fwd) against the CPU oracle
(oracle.conv1d_silu, oracle.mamba_block: f32 arithmetic with bf16 rounding at the same storage
points as the device path). The conv is elementwise-checked (rel_err 1e-4 fp32). The block ends in
a GEMM whose outputs cancel, and a one-ulp flip of any bf16 intermediate propagates, so elementwise
relative error is large even between two correct CPU restatements. The block is held normwise
(max|g - r| / max|r|): <= 2e-2 against the fp32 reference with no storage rounding (the
bf16-storage tolerance) and <= 1e-2 against the oracle that rounds the same intermediates; and
elementwise against the float64 twin of that oracle, to twice the f32 oracle's own elementwise
distance from it (see check_block).
At the BASELINE config-3 size the oracle checks causal prefixes of the first and
last sequences (the block is causal in time and independent across the batch), and the device
output's prefix must equal a device run on that prefix alone, bit for bit."""
import numpy as np
import pytest
import torch

import oracle
from helixml_amd import ssm
from helixml_amd._ffi import InvalidInput, UnsupportedOperation
from tests.util import CW_ULPS, TOL_BF16, TOL_F32, block_inputs, bf16_round, cw_ulps, norm_err, rel_err

pytestmark = pytest.mark.gpu

BF = torch.bfloat16


def to_dev(p, dev):
    bf_names = {"x", "w_in", "w_x", "w_dt", "w_out"}
    return {k: torch.from_numpy(np.ascontiguousarray(v)).to(dev, BF if k in bf_names else torch.float32)
            for k, v in p.items()}


@pytest.mark.parametrize("bt,L,dim,W", [(2, 37, 64, 4), (1, 1, 8, 4), (3, 130, 20, 3), (1, 64, 256, 1),
                                        (2, 9, 12, 2)])
def test_conv1d_silu_f32(dev, bt, L, dim, W):
    rng = np.random.default_rng(bt * 100 + L)
    x = rng.standard_normal((bt, L, dim)).astype(np.float32)
    w = rng.standard_normal((dim, W)).astype(np.float32)
    b = rng.standard_normal(dim).astype(np.float32)
    y = ssm.conv1d_silu(torch.from_numpy(x).to(dev), torch.from_numpy(w).to(dev),
                        torch.from_numpy(b).to(dev))
    err = rel_err(y.cpu().numpy(), oracle.conv1d_silu(x, w, b))
    assert err < TOL_F32, err


def test_conv1d_silu_bf16_strided_rows(dev):
    # x is the first half of a [bt, L, 2*dim] in_proj output, as inside the block
    rng = np.random.default_rng(7)
    bt, L, dim = 2, 70, 96
    xz = bf16_round(rng.standard_normal((bt, L, 2 * dim)).astype(np.float32))
    w = (rng.standard_normal((dim, 4)) * 0.5).astype(np.float32)
    b = rng.standard_normal(dim).astype(np.float32)
    xz_d = torch.from_numpy(xz).to(dev, BF)
    y = ssm.conv1d_silu(xz_d[:, :, :dim], torch.from_numpy(w).to(dev), torch.from_numpy(b).to(dev))
    r = oracle.conv1d_silu(xz[:, :, :dim], w, b)
    g = y.float().cpu().numpy()
    # only the output rounding to bf16 separates the two: half an ulp, 2^-9 relative
    e1, e2 = norm_err(g, r), rel_err(g, bf16_round(r))
    assert e1 <= 2.0 ** -8, e1
    assert e2 < TOL_BF16, e2


def test_conv1d_silu_bf16_long_runs(dev):
    """At config-5 size (16 x 8197 x 1024, a ragged last run) the kernel takes 32-step runs with
    every input row loaded up front; one sequence alone takes 16-step runs. Both give the same
    bits, and stay within the bf16 output rounding of the oracle."""
    rng = np.random.default_rng(8)
    bt, L, dim = 16, 8197, 1024
    x = torch.randn((bt, L, dim), generator=torch.Generator().manual_seed(8)).to(dev, BF)
    w = (rng.standard_normal((dim, 4)) * 0.5).astype(np.float32)
    b = rng.standard_normal(dim).astype(np.float32)
    wd, bd = torch.from_numpy(w).to(dev), torch.from_numpy(b).to(dev)
    y = ssm.conv1d_silu(x, wd, bd)
    for s in (0, bt - 1):
        ys = ssm.conv1d_silu(x[s:s + 1].contiguous(), wd, bd)
        assert torch.equal(ys[0], y[s]), f"sequence {s}: 32-step and 16-step runs differ"
    xs = x[bt - 1].float().cpu().numpy()[None]
    r = oracle.conv1d_silu(xs, w, b)
    g = y[bt - 1:].float().cpu().numpy()
    e1, e2 = norm_err(g, r), rel_err(g, bf16_round(r))
    assert e1 <= 2.0 ** -8, e1
    assert e2 < TOL_BF16, e2


def test_conv1d_rejects_bad_width_and_dim(dev):
    x = torch.zeros((1, 4, 8), device=dev)
    with pytest.raises(UnsupportedOperation):
        ssm.conv1d_silu(x, torch.zeros((8, 5), device=dev))
    with pytest.raises(UnsupportedOperation):
        ssm.conv1d_silu(torch.zeros((1, 4, 6), device=dev), torch.zeros((6, 4), device=dev))


@pytest.mark.parametrize("bt,L,dm,di,r", [(2, 64, 64, 128, 16), (1, 100, 32, 64, 8),
                                          (2, 300, 128, 256, 16), (3, 17, 48, 96, 8),
                                          (2, 60, 64, 2048, 16), (1, 40, 64, 2048, 200),
                                          (2, 37, 64, 256, 32), (1, 130, 96, 128, 64),
                                          (3, 50, 64, 192, 96), (1, 33, 64, 256, 128)])
def test_mamba_block_vs_oracle(dev, bt, L, dm, di, r):
    """(2, 60, 64, 2048, 16) runs x_proj through the narrow kernel (N 48, K 2048), (1, 40, 64, 2048,
    200) split four ways along K (N 232); dt_rank 32, 64, 96 and 128 take dt_proj inside the scan
    (ragged last chunks, a partial channel tile at d_inner 192), the others the separate product."""
    p = block_inputs(bt, L, dm, di, 16, r, 4, seed=bt * 1000 + L)
    y = ssm.mamba_block_fwd(**to_dev(p, dev))
    torch.cuda.synchronize()
    assert y.shape == (bt, L, dm) and y.dtype == BF
    check_block(y.float().cpu().numpy(), p, r)


def check_block(g, p, r, what=""):
    """Normwise: <= 1e-2 against the same-rounding f32 oracle, <= 2e-2 against the fp32 oracle
    with no storage rounding. Elementwise against the float64 twin with the same rounding
    points, componentwise: each output within CW_ULPS bf16 ulps (2^-8) of |y| . |w_out|^T, the
    magnitudes of the terms out_proj sums for it. (The plain relative error, also printed, divides
    the rounding of large terms by a small output where out_proj cancels: a one-ulp flip of a bf16
    intermediate there gives 0.1-0.2 between two correct evaluations.)"""
    ref = oracle.mamba_block(**p, dt_rank=r)
    ref64, terms = oracle.numpy_mamba_block(**p, dt_rank=r, return_terms=True)
    e_same = norm_err(g, ref)
    e_fp32 = norm_err(g, oracle.mamba_block(**p, dt_rank=r, bf16=False))
    e_cw, own_cw = cw_ulps(g, ref64, terms), cw_ulps(ref, ref64, terms)
    print(f"block{what}: normwise {e_same:.3e} (bf16-storage oracle), {e_fp32:.3e} (fp32 oracle); "
          f"componentwise {e_cw:.3f} bf16 ulps of the terms (f32 oracle's own {own_cw:.3f}); "
          f"plain elementwise {rel_err(g, ref64):.3e} (f32 oracle's own {rel_err(ref, ref64):.3e})", flush=True)
    assert e_same <= 1e-2, f"{what} vs bf16-storage oracle: {e_same}"
    assert e_fp32 <= TOL_BF16, f"{what} vs fp32 oracle: {e_fp32}"
    assert e_cw <= CW_ULPS, f"{what} componentwise vs float64 twin: {e_cw} bf16 ulps (own {own_cw})"


def test_mamba_block_class_matches_functional(dev):
    g = torch.Generator().manual_seed(5)
    blk = ssm.MambaBlock(64, d_state=16, d_conv=4, expand=2, device=dev, generator=g)
    x = torch.randn((2, 50, 64), generator=g).to(dev, BF)
    y1 = blk(x)
    y2 = ssm.mamba_block_fwd(x, **blk.parameters())
    assert torch.equal(y1, y2)
    p = {k: v.float().cpu().numpy() for k, v in blk.parameters().items()}
    check_block(y1.float().cpu().numpy(), dict(p, x=x.float().cpu().numpy()), blk.dt_rank)
    # a longer input regrows the kept workspace
    x3 = torch.randn((1, 200, 64), generator=g).to(dev, BF)
    assert torch.equal(blk(x3), ssm.mamba_block_fwd(x3, **blk.parameters()))


def test_mamba_block_errors(dev):
    p = to_dev(block_inputs(1, 8, 16, 32, 16, 8, 4, seed=1), dev)
    small = torch.empty(16, device=dev, dtype=torch.uint8)
    with pytest.raises(InvalidInput):
        ssm.mamba_block_fwd(**p, workspace=small)
    p8 = to_dev(block_inputs(1, 8, 16, 32, 8, 8, 4, seed=1), dev)
    with pytest.raises(UnsupportedOperation):
        ssm.mamba_block_fwd(**p8)


def test_mamba_block_config3_full_size(dev):
    """batch 4, L 4096, d_model 2048, d_inner 4096, N 16, dt_rank 128, k 4."""
    bt, L, dm, di, r = 4, 4096, 2048, 4096, 128
    p = block_inputs(bt, L, dm, di, 16, r, 4, seed=3)
    d = to_dev(p, dev)
    y = ssm.mamba_block_fwd(**d)
    torch.cuda.synchronize()
    assert torch.isfinite(y.float()).all()
    T = 48
    for b in (0, bt - 1):
        pb = dict(p, x=p["x"][b:b + 1, :T])
        yb = ssm.mamba_block_fwd(**dict(d, x=d["x"][b:b + 1, :T].contiguous()))
        torch.cuda.synchronize()
        same = torch.equal(yb[0], y[b, :T])
        assert same, f"prefix of sequence {b} differs from the full run"
        check_block(yb.float().cpu().numpy(), pb, r, f"sequence {b}")
