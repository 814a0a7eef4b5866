"""bf16 matrix-core GEMM (hx_gemm_bf16) against a plain PyTorch fp32 reference of the same op
(the bf16 inputs upcast, matmul in fp32 on the CPU). bf16 output is compared after rounding."""
import numpy as np
import pytest
import torch

from helixml_amd import ssm
from tests.util import norm_err, rel_err

pytestmark = pytest.mark.gpu


def ref(X, W, bias=None, act=0):
    y = X.float().cpu() @ W.float().cpu().T
    if bias is not None:
        y = y + bias.float().cpu()
    if act == 1:
        y = y * torch.sigmoid(y)
    return y.numpy()


@pytest.mark.parametrize("M,N,K", [(128, 128, 32), (256, 384, 512), (100, 70, 40), (1, 1, 8),
                                   (300, 160, 4096), (512, 2048, 256), (129, 257, 264)])
@pytest.mark.parametrize("act", [0, 1])
def test_gemm_fp32_out(dev, M, N, K, act):
    g = torch.Generator().manual_seed(M * 7 + N)
    X = torch.randn(M, K, generator=g).to(torch.bfloat16).to(dev)
    W = (torch.randn(N, K, generator=g) / np.sqrt(K)).to(torch.bfloat16).to(dev)
    b = torch.randn(N, generator=g).to(dev)
    y = ssm.gemm_bf16(X, W, b, act=act, out_dtype=torch.float32)
    torch.cuda.synchronize()
    r = ref(X, W, b, act)
    # fp32 accumulation in a different order than the reference: a K-long dot product can
    # cancel, so the bar is normwise (max abs error / max abs value), sized for K up to 4096
    assert norm_err(y.cpu().numpy(), r) <= 1e-5


def test_gemm_bf16_out_splits_and_strided_input(dev):
    g = torch.Generator().manual_seed(3)
    M, K, N = 200, 256, 160
    Xfull = torch.randn(M, 320, generator=g).to(torch.bfloat16).to(dev)
    X = Xfull[:, 64:64 + K]  # row-strided view (ld = 320)
    W = (torch.randn(N, K, generator=g) / 16).to(torch.bfloat16).to(dev)
    a, b, c = ssm.gemm_bf16(X, W, splits=(128, 144))
    torch.cuda.synchronize()
    r = ref(X, W)
    got = np.concatenate([a.float().cpu().numpy(), b.float().cpu().numpy(), c.float().cpu().numpy()], 1)
    assert a.shape == (M, 128) and b.shape == (M, 16) and c.shape == (M, 16)
    assert rel_err(got, r) <= 2 ** -8  # one bf16 rounding of the output


@pytest.mark.parametrize("M,N,K", [(64, 40, 4), (130, 70, 13), (33, 256, 36)])
def test_gemm_unaligned_rows(dev, M, N, K):
    # K not a multiple of 8: rows are not 16-byte aligned, the element-load variant runs
    g = torch.Generator().manual_seed(K)
    X = torch.randn(M, K, generator=g).to(torch.bfloat16).to(dev)
    W = torch.randn(N, K, generator=g).to(torch.bfloat16).to(dev)
    y = ssm.gemm_bf16(X, W, out_dtype=torch.float32)
    err = norm_err(y.cpu().numpy(), ref(X, W))
    assert err <= 1e-5, err
