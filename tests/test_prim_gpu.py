"""Device primitives (hx_binary_f32, hx_unary_f32, hx_mean_axis_f32, hx_copy_strided_f32,
hx_fill_f32, hx_eye_f32 through helixml_amd.prim) against the oracle's restatement of CpuTensor
(crates/backend-cpu/src/lib.rs) on identical seeded inputs.

Bars: bit-exact for add/sub/mul/div, mul_scalar/add_scalar/neg/abs, sqrt, mean and every copy
(transpose, slice, broadcast_to, stack, cat, fill, eye); max relative error <= 1e-6 (metric in
tests/util.py) for exp/cos/sin/log/silu/sigmoid, where the device math library stands in for the
host libm the reference calls."""
import numpy as np
import pytest
import torch

import oracle
from helixml_amd import prim
from helixml_amd._ffi import InvalidDimension, ShapeMismatch, UnsupportedOperation
from tests.util import rel_err

pytestmark = pytest.mark.gpu

TOL_LIBM = 1e-6


def dev_t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev)


def host(t):
    return t.cpu().numpy()


def bits_equal(g, r):
    g = np.ascontiguousarray(g, np.float32)
    r = np.ascontiguousarray(r, np.float32)
    return g.shape == r.shape and np.array_equal(g.view(np.uint32), r.view(np.uint32))


SIZES = [1, 3, 4, 17, 1000, 65537]


@pytest.mark.parametrize("n", SIZES)
@pytest.mark.parametrize("op", ["add", "sub", "mul", "div"])
def test_binary_bit_exact(dev, op, n):
    rng = np.random.default_rng(n)
    a = rng.standard_normal(n).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    ref = {"add": a + b, "sub": a - b, "mul": a * b, "div": a / b}[op]
    assert bits_equal(host(prim.binary(op, dev_t(a, dev), dev_t(b, dev))), ref)


def test_binary_unaligned_view_and_kat(dev):
    """A 4-byte-offset operand takes the scalar path; the reference's own KAT ones + ones = 2
    (backend-cpu/src/lib.rs:1733-1744)."""
    x = torch.ones(1001, device=dev)
    y = prim.binary("add", x[1:].contiguous(), x[:-1].contiguous())
    assert torch.equal(y, torch.full((1000,), 2.0, device=dev))
    base = torch.arange(1001, device=dev, dtype=torch.float32)
    a = base[1:]  # 4-byte aligned, not 16
    out = prim.binary("mul", a, a)
    assert bits_equal(host(out), host(a) * host(a))


def test_binary_shape_mismatch(dev):
    with pytest.raises(ShapeMismatch):
        prim.binary("add", torch.ones(2, 3, device=dev), torch.ones(3, 2, device=dev))


@pytest.mark.parametrize("n", SIZES)
@pytest.mark.parametrize("op", ["mul_scalar", "add_scalar", "neg", "abs", "sqrt"])
def test_unary_exact_ops(dev, op, n):
    rng = np.random.default_rng(7 + n)
    x = rng.standard_normal(n).astype(np.float32)
    if op == "sqrt":
        x = np.abs(x)
    s = np.float32(0.37)
    g = host(prim.unary(op, dev_t(x, dev), float(s)))
    assert bits_equal(g, oracle.unary(op, x, float(s)))


@pytest.mark.parametrize("op", ["exp", "cos", "sin", "log", "silu", "sigmoid"])
def test_unary_libm_ops(dev, op):
    rng = np.random.default_rng(11)
    x = (rng.standard_normal(100003) * 4).astype(np.float32)
    if op == "log":
        x = np.abs(x) + np.float32(1e-3)
    g = host(prim.unary(op, dev_t(x, dev)))
    r = oracle.unary(op, x)
    e = rel_err(g, r)
    print(f"{op}: max rel err {e:.2e}")
    assert e <= TOL_LIBM


@pytest.mark.parametrize("shape,axis", [
    ((5, 9), 1), ((5, 9), 0), ((3, 1, 16), 1), ((2, 3, 17), 2), ((4, 1000), 1), ((1000, 4), 0),
    ((7,), 0), ((2, 3, 4, 5), 2), ((300, 8), 1), ((64, 33), 1)])
def test_mean_axis_bit_exact(dev, shape, axis):
    rng = np.random.default_rng(sum(shape) + axis)
    x = rng.standard_normal(shape).astype(np.float32)
    g = host(prim.mean(dev_t(x, dev), [axis]))
    assert bits_equal(g, oracle.mean_axis(x, axis))


def test_mean_summation_order(dev):
    """The crafted row whose eight-accumulator sum is 6 and sequential sum 3: the last axis takes
    the fold (6/9), another axis the sequential order (3/9)."""
    row = np.array([1e8, 1, 1, 1, -1e8, 1, 1, 1, 0], np.float32)
    assert host(prim.mean(dev_t(row[None, :], dev), [1]))[0] == np.float32(6) / np.float32(9)
    assert host(prim.mean(dev_t(row[:, None], dev), [0]))[0] == np.float32(3) / np.float32(9)


def test_mean_multiple_dims_and_all(dev):
    rng = np.random.default_rng(5)
    x = rng.standard_normal((3, 4, 10)).astype(np.float32)
    # dims [0, 2]: axis 2 first (the fold), then axis 0 of the [3, 4] result (sequential)
    r = oracle.mean_axis(oracle.mean_axis(x, 2), 0)
    assert bits_equal(host(prim.mean(dev_t(x, dev), [0, 2])), r)
    r_all = oracle.mean_axis(oracle.mean_axis(oracle.mean_axis(x, 2), 1), 0)
    assert bits_equal(host(prim.mean(dev_t(x, dev))), r_all)
    with pytest.raises(InvalidDimension):
        prim.mean(dev_t(x, dev), [3])


@pytest.mark.parametrize("src,dst", [
    ((5,), (3, 5)), ((1,), (1, 6)), ((4, 5), (3, 4, 5)), ((1, 5), (2, 3, 5)),
    ((5,), (2, 3, 5)), ((2, 3, 1), (2, 3, 7)), ((4, 1), (4, 6)), ((2, 3), (1, 1, 2, 3)),
    ((3,), (2, 2, 2, 3)), ((1, 2, 1, 3), (2, 2, 4, 3))])
def test_broadcast_to_matches_reference_index_map(dev, src, dst):
    rng = np.random.default_rng(len(src) * 10 + len(dst))
    x = rng.standard_normal(src).astype(np.float32)
    g = host(prim.broadcast_to(dev_t(x, dev), dst))
    assert bits_equal(g, oracle.broadcast_to(x, dst))


def test_broadcast_to_errors(dev):
    with pytest.raises(ShapeMismatch):
        prim.broadcast_to(torch.ones(4, device=dev), [3, 5])
    with pytest.raises(ShapeMismatch):  # [R] -> [R, C]: the compatibility check (lib.rs:1373-1380)
        prim.broadcast_to(torch.ones(3, device=dev), [3, 4])  # runs before the repeat-columns branch
    with pytest.raises(ShapeMismatch):  # a size-1 vector to [R, C], R, C > 1 (lib.rs:1420-1425)
        prim.broadcast_to(torch.ones(1, device=dev), [3, 5])
    with pytest.raises(ShapeMismatch):
        prim.broadcast_to(torch.ones(2, 3, device=dev), [3])


@pytest.mark.parametrize("shape,d0,d1", [((3, 5), 0, 1), ((2, 3, 4), 0, 2), ((2, 3, 4), 1, 1),
                                         ((64, 129), 1, 0), ((2, 3, 4, 5), 1, 3)])
def test_transpose(dev, shape, d0, d1):
    x = np.random.default_rng(1).standard_normal(shape).astype(np.float32)
    assert bits_equal(host(prim.transpose(dev_t(x, dev), d0, d1)), oracle.transpose(x, d0, d1))
    with pytest.raises(InvalidDimension):
        prim.transpose(dev_t(x, dev), 0, len(shape))


def test_slice_2d_and_errors(dev):
    x = np.random.default_rng(2).standard_normal((7, 9)).astype(np.float32)
    for start, end in [([0, 0], [7, 9]), ([2, 3], [5, 4]), ([6, 0], [7, 9]), ([0, 8], [7, 9])]:
        assert bits_equal(host(prim.slice(dev_t(x, dev), start, end)), oracle.slice2d(x, start, end))
    with pytest.raises(ShapeMismatch):
        prim.slice(dev_t(x, dev), [0], [1])
    with pytest.raises(InvalidDimension):
        prim.slice(dev_t(x, dev), [3, 0], [3, 2])
    with pytest.raises(UnsupportedOperation):
        prim.slice(torch.ones(2, 2, 2, device=dev), [0, 0, 0], [1, 1, 1])


@pytest.mark.parametrize("shape,dim,count", [((5,), 1, 4), ((5,), 0, 3), ((2, 3), 2, 3),
                                             ((2, 3, 4), 1, 2), ((2, 3, 2, 2), 2, 3),
                                             ((2, 1, 3, 2), 0, 2), ((2, 2, 2, 2), 4, 2)])
def test_stack(dev, shape, dim, count):
    rng = np.random.default_rng(len(shape) + dim)
    xs = [rng.standard_normal(shape).astype(np.float32) for _ in range(count)]
    g, field = prim.stack([dev_t(x, dev) for x in xs], dim)
    r, rfield = oracle.stack(xs, dim)
    assert field == rfield and bits_equal(host(g).reshape(-1), r.reshape(-1))


def test_stack_shape_field_quirk(dev):
    """stack(., 1) of per-step [d_model] vectors (S4Block::forward_ssm, ssm.rs:185): the data are
    the steps back to back ([L, d_model] in memory) while the shape field reads [d_model, L]."""
    steps = [np.full(3, t, np.float32) for t in range(4)]
    g, field = prim.stack([dev_t(s, dev) for s in steps], 1)
    assert field == [3, 4]
    assert np.array_equal(host(g).reshape(-1), np.repeat(np.arange(4, dtype=np.float32), 3))


def test_stack_and_cat_errors(dev):
    a, b = torch.ones(3, device=dev), torch.ones(4, device=dev)
    with pytest.raises(UnsupportedOperation):
        prim.stack([], 0)
    with pytest.raises(ShapeMismatch):
        prim.stack([a, b], 0)
    assert torch.equal(prim.cat([a, b], 0), torch.ones(7, device=dev))
    with pytest.raises(UnsupportedOperation):
        prim.cat([torch.ones(2, 2, device=dev)] * 2, 0)
    with pytest.raises(InvalidDimension):
        prim.cat([a, b], 1)


def test_cat_1d(dev):
    rng = np.random.default_rng(3)
    xs = [rng.standard_normal(n).astype(np.float32) for n in (5, 1, 16, 7)]
    assert bits_equal(host(prim.cat([dev_t(x, dev) for x in xs], 0)), oracle.cat1d(xs))


def test_fill_and_eye(dev):
    assert torch.equal(prim.fill([3, 5], 1.5, dev), torch.full((3, 5), 1.5, device=dev))
    assert torch.equal(prim.fill([4097], 0.0, dev), torch.zeros(4097, device=dev))
    assert torch.equal(prim.eye(7, dev), torch.eye(7, device=dev))


def test_rmsnorm_composite_bit_exact(dev):
    """RMSNorm::forward (crates/nn/src/lib.rs:258-285) spelled with the primitives —
    x*x, mean(last), + eps, sqrt, reshape, broadcast_to, div, broadcast weight, mul — equals the
    oracle's restatement bit for bit (eps' = eps)."""
    rng = np.random.default_rng(9)
    x = rng.standard_normal((37, 64)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(64)).astype(np.float32)
    X, W = dev_t(x, dev), dev_t(w, dev)
    ms = prim.mean(prim.binary("mul", X, X), [1])
    rms = prim.unary("sqrt", prim.binary("add", ms, prim.fill(ms.shape, 1e-5, dev)))
    rms_b = prim.broadcast_to(rms.reshape(37, 1), [37, 64])
    y = prim.binary("mul", prim.binary("div", X, rms_b), prim.broadcast_to(W, [37, 64]))
    assert bits_equal(host(y), oracle.rmsnorm_ref(x, w, 1e-5))
