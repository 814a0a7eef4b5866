"""hx_selective_scan_fwd_noalloc (device-resident scratch, no allocation) against
hx_selective_scan_fwd_ws (caller workspace) through the C ABI: identical bits on two calls in a
row on the segmented long-sequence path, the second with a smaller input (the scratch keeps the
first call's contents), plus the size limit."""
import ctypes

import pytest
import torch

from helixml_amd import _ffi

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 8 << 20


def _inputs(bt, L, dim, seed, dtype):
    g = torch.Generator(device="cuda:0")
    g.manual_seed(seed)
    dev = "cuda:0"
    n = lambda *s: torch.randn(*s, device=dev, generator=g)  # noqa: E731
    return dict(
        u=n(bt, L, dim).to(dtype), delta=(n(bt, L, dim) * 0.5 - 4.0).to(dtype),
        A=-torch.arange(1, 17, device=dev, dtype=torch.float32).repeat(dim, 1).contiguous(),
        B=n(bt, L, 16).to(dtype), C=n(bt, L, 16).to(dtype), D=n(dim),
        z=n(bt, L, dim).to(dtype), dt_bias=n(dim) * 0.1, init=n(bt, dim, 16) * 0.1)


def _p(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _run(name, x, bt, L, dim, dtype, ws=None):
    out = torch.full((bt, L, dim), float("nan"), device="cuda:0", dtype=dtype)
    last = torch.full((bt, dim, 16), float("nan"), device="cuda:0", dtype=torch.float32)
    code = _ffi.HX_F32 if dtype == torch.float32 else _ffi.HX_BF16
    args = [bt, L, dim, 16, code, 1, _p(x["u"]), _p(x["delta"]), _p(x["A"]), _p(x["B"]),
            _p(x["C"]), _p(x["D"]), _p(x["z"]), _p(x["dt_bias"]), _p(out), _p(x["init"]), _p(last)]
    if name == "hx_selective_scan_fwd_ws":
        args += [_p(ws) if ws is not None else None, ws.numel() if ws is not None else 0]
    _ffi.call(name, *args, None)
    torch.cuda.synchronize()
    return out, last


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_noalloc_matches_workspace_entry_two_calls(dev, dtype):
    L_ = _ffi.lib()
    code = _ffi.HX_F32 if dtype == torch.float32 else _ffi.HX_BF16
    # second call smaller than the first; both take the segmented path (scratch in use)
    for i, (bt, L, dim) in enumerate([(1, 32768, 2048), (1, 8192, 512)]):
        need = int(L_.hx_selective_scan_workspace_size(bt, L, dim, 16, code))
        print(f"case no-alloc call {i}: {bt}x{L}x{dim} {dtype} scratch {need} B", flush=True)
        assert 0 < need <= SCRATCH_BYTES
        x = _inputs(bt, L, dim, seed=100 + i, dtype=dtype)
        ws = torch.empty(need, device=dev, dtype=torch.uint8)
        ref_out, ref_last = _run("hx_selective_scan_fwd_ws", x, bt, L, dim, dtype, ws)
        out, last = _run("hx_selective_scan_fwd_noalloc", x, bt, L, dim, dtype)
        assert not torch.isnan(ref_out.float()).any()
        assert torch.equal(out.view(torch.int16) if dtype == torch.bfloat16 else out.view(torch.int32),
                           ref_out.view(torch.int16) if dtype == torch.bfloat16 else ref_out.view(torch.int32))
        assert torch.equal(last.view(torch.int32), ref_last.view(torch.int32))


def test_noalloc_unsegmented_matches_plain_entry(dev):
    """A shape that fills the GPU without segments uses no scratch: same bits as
    hx_selective_scan_fwd."""
    bt, L, dim = 2, 300, 192
    x = _inputs(bt, L, dim, seed=7, dtype=torch.float32)
    ref_out, ref_last = _run("hx_selective_scan_fwd", x, bt, L, dim, torch.float32)
    out, last = _run("hx_selective_scan_fwd_noalloc", x, bt, L, dim, torch.float32)
    assert torch.equal(out.view(torch.int32), ref_out.view(torch.int32))
    assert torch.equal(last.view(torch.int32), ref_last.view(torch.int32))


def test_noalloc_rejects_scratch_beyond_limit(dev):
    """Forcing 4096 segments at 1 x 65536 x 2048 asks for ~1.1 GB of scratch: rejected before any
    launch with UnsupportedOperation."""
    from helixml_amd import ssm
    ssm.set_scan_segments(4096)
    try:
        need = int(_ffi.lib().hx_selective_scan_workspace_size(1, 65536, 2048, 16, _ffi.HX_F32))
        assert need > SCRATCH_BYTES
        rc = _ffi.lib().hx_selective_scan_fwd_noalloc(1, 65536, 2048, 16, _ffi.HX_F32, 1,
                                                      *([None] * 11), None)
        assert rc == _ffi.UnsupportedOperation.status
        assert "scratch" in _ffi.last_error()
    finally:
        ssm.set_scan_segments(0)
