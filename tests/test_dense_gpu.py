"""Parity of the fp32 dense kernels (hx_linear_f32, hx_matmul_f32) and the exported
nn::MambaBlock MLP composition (crates/nn/src/lib.rs:888-906) against the CPU oracle."""
import numpy as np
import pytest
import torch

import oracle
from helixml_amd import ShapeMismatch, ssm
from tests.util import TOL_F32, rel_err

pytestmark = pytest.mark.gpu
F = np.float32


def dv(x, dev):
    return None if x is None else torch.from_numpy(np.ascontiguousarray(x)).to(dev)


@pytest.mark.parametrize("R,IN,OUT", [(100, 64, 128), (1, 1, 1), (65, 70, 33), (300, 512, 256)])
@pytest.mark.parametrize("act", [0, 1])
def test_linear(dev, R, IN, OUT, act):
    rng = np.random.default_rng(R + IN + OUT)
    X = rng.uniform(-1, 1, (R, IN)).astype(F)
    W = (rng.standard_normal((OUT, IN)) * np.sqrt(2.0 / IN)).astype(F)
    b = rng.standard_normal(OUT).astype(F)
    g = ssm.linear(dv(X, dev), dv(W, dev), dv(b, dev), act=act).cpu().numpy()
    assert rel_err(g, oracle.linear(X, W, b, act)) <= TOL_F32


@pytest.mark.parametrize("M,K,N", [(64, 64, 64), (2, 3, 4), (37, 129, 65)])
def test_matmul(dev, M, K, N):
    rng = np.random.default_rng(M * K)
    A = rng.standard_normal((M, K)).astype(F)
    B = rng.standard_normal((K, N)).astype(F)
    assert rel_err(ssm.matmul(dv(A, dev), dv(B, dev)).cpu().numpy(), oracle.matmul(A, B)) <= TOL_F32


def test_matmul_reference_kat(dev):
    # backend-cpu/src/lib.rs:1747-1758
    y = ssm.matmul(torch.ones(2, 3, device=dev), torch.ones(3, 4, device=dev)).cpu().numpy()
    assert np.all(np.abs(y - 3.0) < 1e-6)


def test_matmul_mismatch_error(dev):
    # backend-cpu/tests/integration_tests.rs:101-112: mismatched inner dims is a ShapeMismatch
    with pytest.raises(ShapeMismatch):
        ssm.matmul(torch.ones(2, 3, device=dev), torch.ones(4, 2, device=dev))


def test_exported_mamba_mlp_config1(dev):
    # README SSM example shape: [100, 64], expand 2
    rng = np.random.default_rng(1)
    X = rng.uniform(-1, 1, (100, 64)).astype(F)
    Wg = (rng.standard_normal((128, 64)) * np.sqrt(2 / 64)).astype(F)
    Wo = (rng.standard_normal((64, 128)) * np.sqrt(2 / 128)).astype(F)
    bg, bo = np.zeros(128, F), np.zeros(64, F)
    h = ssm.linear(dv(X, dev), dv(Wg, dev), dv(bg, dev), act=1)
    g = ssm.linear(h, dv(Wo, dev), dv(bo, dev)).cpu().numpy()
    assert rel_err(g, oracle.mamba_mlp(X, Wg, bg, Wo, bo)) <= TOL_F32


@pytest.mark.parametrize("R,IN,OUT", [(100, 64, 128), (65, 70, 33)])
def test_linear_and_matmul_bit_exact(dev, R, IN, OUT):
    """Unfused products summed over k ascending from 0.0, then + bias: bit-identical to
    CpuTensor::matmul (backend-cpu/src/lib.rs:659-667) and Linear::forward (nn/src/lib.rs:125-130)."""
    rng = np.random.default_rng(R * IN)
    X = rng.uniform(-1, 1, (R, IN)).astype(F)
    W = rng.standard_normal((OUT, IN)).astype(F)
    b = rng.standard_normal(OUT).astype(F)
    assert np.array_equal(ssm.linear(dv(X, dev), dv(W, dev), dv(b, dev)).cpu().numpy(), oracle.linear(X, W, b))
    Wt = np.ascontiguousarray(W.T)
    assert np.array_equal(ssm.matmul(dv(X, dev), dv(Wt, dev)).cpu().numpy(), oracle.matmul(X, Wt))
