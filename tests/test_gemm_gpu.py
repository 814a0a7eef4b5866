"""bf16 matrix-core GEMM (hx_gemm_bf16) against a plain PyTorch fp32 reference of the same op
(the bf16 inputs upcast, matmul in fp32 on the CPU). bf16 output is compared after rounding."""
import numpy as np
import pytest
import torch

from helixml_amd import ssm
from helixml_amd._ffi import InvalidInput, UnsupportedOperation
from tests.util import bf16_round, norm_err, rel_err

pytestmark = pytest.mark.gpu


def ref(X, W, bias=None, act=0):
    y = X.float().cpu() @ W.float().cpu().T
    if bias is not None:
        y = y + bias.float().cpu()
    if act == 1:
        y = y * torch.sigmoid(y)
    return y.numpy()


@pytest.mark.parametrize("M,N,K", [(128, 128, 32), (256, 384, 512), (100, 70, 40), (1, 1, 8),
                                   (300, 160, 4096), (512, 2048, 256), (129, 257, 264),
                                   (256, 2048, 512), (96, 96, 4104)])
@pytest.mark.parametrize("act", [0, 1])
def test_gemm_fp32_out(dev, M, N, K, act):
    """Default kernel choice. (256, 2048, 512) is the decode in_proj shape: the small-M kernel's
    64-wide tiles with 8-wave blocks (256 blocks, one per CU); (96, 96, 4104) its 32-wide 8-wave
    form with K past one round of loads per wave and a last piece past K (masked)."""
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


@pytest.fixture
def gemm_kernel(dev, request):
    ssm.set_gemm_kernel(request.param)
    yield request.param
    ssm.set_gemm_kernel(0)


@pytest.mark.parametrize("gemm_kernel", [1, 3, 4, 5, 6, 7, 8], indirect=True)
@pytest.mark.parametrize("M,N,K", [(512, 256, 512), (300, 200, 136), (257, 129, 64), (1024, 2048, 1024),
                                   (100, 72, 1000), (256, 64, 1024), (33, 40, 24), (300, 260, 192),
                                   (600, 136, 128)])
@pytest.mark.parametrize("act", [0, 1])
def test_gemm_tile_kernels_fp32_out(dev, gemm_kernel, M, N, K, act):
    """Each tile kernel (128 x 128 x 32, the small-M kernel's 32 x 32 / 32 x 64 tiles with K split
    over 4 waves, 256 x 128 x 64 direct-to-LDS, 256 x 256, the narrow 64-row kernel for N <= 256)
    on aligned and ragged shapes; the direct-to-LDS kernels take the shapes with K % 64 (or 32)
    == 0 (1, 2, 3 and more K tiles) and fall back on the others."""
    g = torch.Generator().manual_seed(M + N + K)
    X = torch.randn(M, K, generator=g).to(torch.bfloat16).to(dev)
    W = (torch.randn(N, K, generator=g) / np.sqrt(K)).to(torch.bfloat16).to(dev)
    b = torch.randn(N, generator=g).to(dev)
    y = ssm.gemm_bf16(X, W, b, act=act, out_dtype=torch.float32)
    torch.cuda.synchronize()
    err = norm_err(y.cpu().numpy(), ref(X, W, b, act))
    assert err <= 1e-5, err


@pytest.mark.parametrize("gemm_kernel", [1, 3, 4, 5, 6, 7, 8], indirect=True)
@pytest.mark.parametrize("splits", [(128, 144), (100, 133), (8, 16)])
def test_gemm_tile_kernels_splits_bf16(dev, gemm_kernel, splits):
    """Column splits on vector boundaries and straddling them (100, 133 are not multiples of 8)."""
    g = torch.Generator().manual_seed(sum(splits))
    M, K, N = 520, 256, 200
    X = torch.randn(M, K, generator=g).to(torch.bfloat16).to(dev)
    W = (torch.randn(N, K, generator=g) / 16).to(torch.bfloat16).to(dev)
    parts = ssm.gemm_bf16(X, W, splits=splits)
    torch.cuda.synchronize()
    got = np.concatenate([p.float().cpu().numpy() for p in parts], 1)
    err = rel_err(got, bf16_round(ref(X, W)))
    assert err <= 2 ** -7, err  # within one bf16 ulp of the rounded reference


@pytest.mark.parametrize("gemm_kernel", [1, 3, 4, 5, 6, 7, 8], indirect=True)
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
def test_gemm_accumulate_into_output(dev, gemm_kernel, out_dtype):
    """act bit 1: Y += X . W^T (the residual add of a pre-norm layer)."""
    g = torch.Generator().manual_seed(77)
    M, K, N = 600, 512, 384
    X = torch.randn(M, K, generator=g).to(torch.bfloat16).to(dev)
    W = (torch.randn(N, K, generator=g) / np.sqrt(K)).to(torch.bfloat16).to(dev)
    Y0 = torch.randn(M, N, generator=g).to(dev).to(out_dtype)
    Y = Y0.clone()
    from helixml_amd import _ffi
    od = _ffi.HX_F32 if out_dtype == torch.float32 else _ffi.HX_BF16
    _ffi.call("hx_gemm_bf16", M, N, K, X.data_ptr(), K, W.data_ptr(), K, None, 2, od,
              Y.data_ptr(), N, N, None, 0, N, None, 0, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    r = Y0.float().cpu().numpy() + ref(X, W)
    err = norm_err(Y.float().cpu().numpy(), r)
    assert err <= (1e-5 if out_dtype == torch.float32 else 2 ** -8), err


@pytest.mark.parametrize("gemm_kernel", [0, 5, 6, 8], indirect=True)
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("M,N,K", [(512, 512, 256), (700, 520, 64), (1024, 768, 1088)])
def test_gemm_whole_tile_stores(dev, gemm_kernel, out_dtype, M, N, K):
    """No bias, no activation: the 256 x 256 kernel's whole-tile epilogue (interior 128 x 128
    wave tiles) beside the guarded one (edge tiles), for 1, 2 and 17 K tiles."""
    g = torch.Generator().manual_seed(M * 3 + N + K)
    X = torch.randn(M, K, generator=g).to(torch.bfloat16).to(dev)
    W = (torch.randn(N, K, generator=g) / np.sqrt(K)).to(torch.bfloat16).to(dev)
    y = ssm.gemm_bf16(X, W, out_dtype=out_dtype)
    torch.cuda.synchronize()
    r = ref(X, W)
    if out_dtype == torch.float32:
        assert norm_err(y.cpu().numpy(), r) <= 1e-5
    else:
        assert rel_err(y.float().cpu().numpy(), bf16_round(r)) <= 2 ** -7


@pytest.mark.parametrize("M,N,K,S", [(300, 160, 4096, 4), (1000, 48, 2048, 2), (257, 64, 1024, 16),
                                     (64, 300, 512, 8)])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
def test_gemm_splitk(dev, M, N, K, S, out_dtype):
    """hx_gemm_bf16_splitk: K in S slices, fp32 partials summed in slice order, then the usual
    epilogue (bias, SiLU, column split)."""
    g = torch.Generator().manual_seed(M + N + K + S)
    X = torch.randn(M, K, generator=g).to(torch.bfloat16).to(dev)
    W = (torch.randn(N, K, generator=g) / np.sqrt(K)).to(torch.bfloat16).to(dev)
    b = torch.randn(N, generator=g).to(dev)
    if out_dtype == torch.float32:
        y = ssm.gemm_bf16(X, W, b, act=1, out_dtype=out_dtype, k_splits=S)
        torch.cuda.synchronize()
        assert norm_err(y.cpu().numpy(), ref(X, W, b, 1)) <= 1e-5
    else:
        parts = ssm.gemm_bf16(X, W, splits=(N // 3, N // 2), k_splits=S)
        torch.cuda.synchronize()
        got = np.concatenate([p.float().cpu().numpy() for p in parts], 1)
        assert rel_err(got, bf16_round(ref(X, W))) <= 2 ** -7


def test_gemm_splitk_rejects(dev):
    X = torch.zeros(64, 96, device=dev, dtype=torch.bfloat16)
    W = torch.zeros(32, 96, device=dev, dtype=torch.bfloat16)
    with pytest.raises(UnsupportedOperation):
        ssm.gemm_bf16(X, W, k_splits=2)  # K = 96 is not a multiple of 128
    from helixml_amd import _ffi
    X2 = torch.zeros(64, 128, device=dev, dtype=torch.bfloat16)
    W2 = torch.zeros(32, 128, device=dev, dtype=torch.bfloat16)
    Y = torch.empty(64, 32, device=dev)
    ws = torch.empty(16, device=dev)
    with pytest.raises(InvalidInput):  # workspace smaller than 2 * 64 * 32 floats
        _ffi.call("hx_gemm_bf16_splitk", 64, 32, 128, X2.data_ptr(), 128, W2.data_ptr(), 128, None, 0,
                  _ffi.HX_F32, Y.data_ptr(), 32, 32, None, 0, 32, None, 0, 2, ws.data_ptr(), 64, None)


@pytest.mark.parametrize("gemm_kernel", [4, 5, 8], indirect=True)
@pytest.mark.parametrize("M,N,K", [(2048, 512, 64), (8192, 1024, 256), (12288, 512, 128)])
def test_gemm_grouped_tile_order(dev, gemm_kernel, M, N, K):
    """Grids whose tiles split evenly into whole row panels per XCD take the grouped tile order
    (groups of up to 4 row panels; 12288 x 512 gives each XCD 6 panels of 256 rows: a group of 4
    and one of 2) in the 256 x 256 kernel and the 256 x 128 kernel: every output tile is written
    (the output starts as NaN) and matches the fp32 reference."""
    from helixml_amd import _ffi
    g = torch.Generator().manual_seed(M + N + K)
    X = torch.randn(M, K, generator=g).to(torch.bfloat16).to(dev)
    W = (torch.randn(N, K, generator=g) / np.sqrt(K)).to(torch.bfloat16).to(dev)
    y = torch.full((M, N), float("nan"), device=dev)
    _ffi.call("hx_gemm_bf16", M, N, K, X.data_ptr(), K, W.data_ptr(), K, None, 0, _ffi.HX_F32,
              y.data_ptr(), N, N, None, 0, N, None, 0, None)
    torch.cuda.synchronize()
    yh = y.cpu().numpy()
    assert not np.isnan(yh).any()
    assert norm_err(yh, ref(X, W)) <= 1e-5


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("M,N,K", [(2000, 160, 4096), (333, 64, 1024), (64, 192, 2048), (7, 1, 1024),
                                   (130, 250, 1088), (97, 150, 1024)])
def test_gemm_narrow_kernel(dev, out_dtype, M, N, K):
    """The narrow kernel (64-row tiles holding every column, the x_proj shapes) on its own
    (kernel 7) and as the automatic choice: the block's dt_lo | B | C splits, bias, accumulate,
    ragged M and N (N 150 within a 192-column tile); its fp32 sums are the 256 x 128
    direct-to-LDS kernel's bit for bit (both add
    the same 32 x 32 x 16 MFMA products with K ascending)."""
    g = torch.Generator().manual_seed(M + N + K)
    X = torch.randn(M, K, generator=g).to(torch.bfloat16).to(dev)
    W = (torch.randn(N, K, generator=g) / np.sqrt(K)).to(torch.bfloat16).to(dev)
    b = torch.randn(N, generator=g).to(dev)
    r = ref(X, W, b)
    try:
        ssm.set_gemm_kernel(7)
        y7 = ssm.gemm_bf16(X, W, b, out_dtype=out_dtype)
        s1, s2 = max(1, N // 5), max(1, N // 5) + (N > 2)
        parts = ssm.gemm_bf16(X, W, b, splits=(s1, s2), out_dtype=out_dtype) if N > 2 else None
        ssm.set_gemm_kernel(4)
        y4 = ssm.gemm_bf16(X, W, b, out_dtype=torch.float32)
        ssm.set_gemm_kernel(7)
        y7f = ssm.gemm_bf16(X, W, b, out_dtype=torch.float32)
    finally:
        ssm.set_gemm_kernel(0)
    y0 = ssm.gemm_bf16(X, W, b, out_dtype=out_dtype)
    torch.cuda.synchronize()
    if out_dtype == torch.float32:
        assert norm_err(y7.cpu().numpy(), r) <= 1e-5
    else:
        assert rel_err(y7.float().cpu().numpy(), bf16_round(r)) <= 2 ** -7
    if N <= 192 and K >= 1024:  # the automatic choice for this weight shape
        assert torch.equal(y0, y7)
    if K % 64 == 0:
        assert torch.equal(y7f, y4), "narrow and direct-to-LDS sums differ"
    if parts is not None:
        got = torch.cat([p.float() for p in parts], 1)
        assert torch.equal(got, y7.float())
    # accumulate into the output (act bit 1)
    from helixml_amd import _ffi
    Y0 = torch.randn(M, N, generator=g).to(dev).to(out_dtype)
    Y = Y0.clone()
    od = _ffi.HX_F32 if out_dtype == torch.float32 else _ffi.HX_BF16
    _ffi.call("hx_gemm_bf16", M, N, K, X.data_ptr(), K, W.data_ptr(), K, None, 2, od,
              Y.data_ptr(), N, N, None, 0, N, None, 0, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    err = norm_err(Y.float().cpu().numpy(), Y0.float().cpu().numpy() + ref(X, W))
    assert err <= (1e-5 if out_dtype == torch.float32 else 2 ** -8), err


@pytest.mark.parametrize("gemm_kernel", [0, 4, 5, 6, 7, 8], indirect=True)
def test_gemm_empty_k_is_bias(dev, gemm_kernel):
    """K == 0 gives Y = bias (zeros without one) on every kernel choice: the tile kernels, which
    load whole K tiles, hand it to the guarded 128 x 128 kernel; split-K rejects it."""
    from helixml_amd import _ffi
    M, N = 300, 200
    X = torch.zeros(M, 8, device=dev, dtype=torch.bfloat16)  # 16-byte rows: the vector paths' layout
    W = torch.zeros(N, 8, device=dev, dtype=torch.bfloat16)
    b = torch.randn(N, device=dev)
    Y = torch.full((M, N), 7.0, device=dev)
    s = torch.cuda.current_stream().cuda_stream
    _ffi.call("hx_gemm_bf16", M, N, 0, X.data_ptr(), 8, W.data_ptr(), 8, b.data_ptr(), 0, _ffi.HX_F32,
              Y.data_ptr(), N, N, None, 0, N, None, 0, s)
    torch.cuda.synchronize()
    assert torch.equal(Y, b.expand(M, N))
    ws = torch.empty(2 * M * N, device=dev)
    with pytest.raises(UnsupportedOperation):
        _ffi.call("hx_gemm_bf16_splitk", M, N, 0, X.data_ptr(), 8, W.data_ptr(), 8, None, 0, _ffi.HX_F32,
                  Y.data_ptr(), N, N, None, 0, N, None, 0, 2, ws.data_ptr(), ws.numel() * 4, s)


@pytest.mark.parametrize("gemm_kernel", [0, 1, 3, 4, 5, 6, 7, 8], indirect=True)
@pytest.mark.parametrize("scale", [0, -130])
def test_gemm_bf16_output_rounds_to_nearest_even(dev, gemm_kernel, scale):
    """bf16 outputs are the round-to-nearest-even of the f32 sums, ties to even included, bit for
    bit. Integer operands in [-3, 3] make every product and partial sum exact in f32 (|sum| <=
    9216), whatever the summation order, so the sums are known exactly; most need rounding to 8
    significant bits and many sit on a tie. Scaled by 2^-130 (each operand by 2^-65) the sums below
    16 in magnitude become f32 subnormals, which must round the same way."""
    g = torch.Generator().manual_seed(11)
    M, N, K = 256, 128, 1024
    Xi = torch.randint(-3, 4, (M, K), generator=g).float()
    Wi = torch.randint(-3, 4, (N, K), generator=g).float()
    exact = (Xi.double() @ Wi.double().T) * 2.0 ** scale  # exact: integer sums below 2^24
    s = 2.0 ** (scale // 2)
    X = (Xi * s).to(torch.bfloat16).to(dev)
    W = (Wi * s).to(torch.bfloat16).to(dev)
    y = ssm.gemm_bf16(X, W, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    want = bf16_round(exact.float().numpy())
    got = y.float().cpu().numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), \
        f"{int((got != want).sum())} of {got.size} outputs differ from round-to-nearest-even"


@pytest.mark.parametrize("M,N,K", [(4096, 4300, 64), (2304, 8192, 192), (3000, 6000, 1088)])
def test_gemm_persistent_matches_one_tile_per_block(dev, M, N, K):
    """The persistent 256 x 256 kernel (kernel 8: one block per CU walks its tiles, the K-tile ring
    runs on across tiles) gives the one-tile-per-block kernel's bits on grids with more tiles than
    CUs (1, 3 and 17 K tiles per tile, ragged edges): fp32 out with bias and SiLU, bf16 column
    splits, and accumulation into fp32 and bf16 outputs."""
    from helixml_amd import _ffi
    g = torch.Generator().manual_seed(M + N + K)
    X = torch.randn(M, K, generator=g).to(torch.bfloat16).to(dev)
    W = (torch.randn(N, K, generator=g) / np.sqrt(K)).to(torch.bfloat16).to(dev)
    b = torch.randn(N, generator=g).to(dev)
    Y0 = {dt: torch.randn(M, N, generator=g).to(dev).to(dt) for dt in (torch.float32, torch.bfloat16)}
    s = torch.cuda.current_stream().cuda_stream

    def run(kernel):
        ssm.set_gemm_kernel(kernel)
        try:
            out = [ssm.gemm_bf16(X, W, b, act=1, out_dtype=torch.float32),
                   ssm.gemm_bf16(X, W, out_dtype=torch.float32)]
            out += list(ssm.gemm_bf16(X, W, splits=(N // 3 // 8 * 8, N // 2)))
            for dt, y0 in Y0.items():
                y = y0.clone()
                od = _ffi.HX_F32 if dt == torch.float32 else _ffi.HX_BF16
                _ffi.call("hx_gemm_bf16", M, N, K, X.data_ptr(), K, W.data_ptr(), K, None, 2, od,
                          y.data_ptr(), N, N, None, 0, N, None, 0, s)
                out.append(y)
            torch.cuda.synchronize()
            return out
        finally:
            ssm.set_gemm_kernel(0)

    got, want = run(8), run(5)
    for i, (a, c) in enumerate(zip(got, want)):
        assert torch.equal(a, c), f"output {i} differs from the one-tile-per-block kernel"
    assert norm_err(got[0].cpu().numpy(), ref(X, W, b, 1)) <= 1e-5


@pytest.mark.parametrize("kernel", [5, 8])
def test_gemm_pointer_loads_past_2gib(dev, kernel):
    """The 256 x 256 kernels load their tiles with 32-bit buffer offsets where every byte offset
    into X and W stays below 2^31, and with 64-bit pointer loads otherwise. X here is exactly 2 GiB
    (131072 x 8192 bf16), so the whole product takes the pointer form; its first and last 256 rows
    must be the bits of the same kernel run on those rows alone (the buffer form: the same MFMA
    products in the same order)."""
    M, N, K = 131072, 256, 8192
    g = torch.Generator(device=dev).manual_seed(kernel)
    X = torch.randn(M, K, device=dev, generator=g).to(torch.bfloat16)
    W = (torch.randn(N, K, device=dev, generator=g) / np.sqrt(K)).to(torch.bfloat16)
    print(f"case gemm {M}x{N}x{K} kernel {kernel} (2 GiB X)", flush=True)
    ssm.set_gemm_kernel(kernel)
    try:
        Y = ssm.gemm_bf16(X, W, out_dtype=torch.float32)
        head = ssm.gemm_bf16(X[:256].contiguous(), W, out_dtype=torch.float32)
        tail = ssm.gemm_bf16(X[M - 256:].contiguous(), W, out_dtype=torch.float32)
        torch.cuda.synchronize()
    finally:
        ssm.set_gemm_kernel(0)
    assert torch.equal(Y[:256], head)
    assert torch.equal(Y[M - 256:], tail)
    assert norm_err(tail.cpu().numpy(), ref(X[M - 256:], W)) <= 1e-5
    del X, Y
