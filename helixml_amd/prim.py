"""CpuTensor's primitives on device tensors through the C ABI (hx_binary_f32, hx_unary_f32,
hx_mean_axis_f32, hx_copy_strided_f32, hx_fill_f32, hx_eye_f32) — the Python twin of the C++
HipTensor operations (include/helix/helix.hpp), with the reference's semantics and error variants
(crates/backend-cpu/src/lib.rs). torch supplies device memory only; every value is computed by the
HIP kernels. fp32, row-major contiguous tensors."""
from __future__ import annotations

import ctypes

import torch

from . import _ffi
from ._ffi import InvalidDimension, ShapeMismatch, UnsupportedOperation

BINARY = {"add": 0, "sub": 1, "mul": 2, "div": 3}
UNARY = {"exp": 0, "cos": 1, "sin": 2, "sqrt": 3, "silu": 4, "neg": 5, "mul_scalar": 6,
         "add_scalar": 7, "abs": 8, "log": 9, "sigmoid": 10}
MAX_DIMS = 8


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def _need_f32(t):
    if t.dtype != torch.float32 or not t.is_cuda or not t.is_contiguous():
        raise _ffi.DTypeMismatch("expected a contiguous float32 device tensor")


def binary(op: str, a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """CpuTensor::add/sub/mul/div (lib.rs:570-632): equal shapes, else ShapeMismatch."""
    if tuple(a.shape) != tuple(b.shape):
        raise ShapeMismatch(f"Shape mismatch: expected {list(a.shape)}, got {list(b.shape)}")
    _need_f32(a)
    _need_f32(b)
    y = torch.empty_like(a)
    _ffi.call("hx_binary_f32", BINARY[op], a.numel(), _p(a), _p(b), _p(y), None)
    return y


def unary(op: str, x: torch.Tensor, scalar: float = 0.0) -> torch.Tensor:
    """exp/cos/sin/sqrt/silu/neg/mul_scalar/add_scalar/abs/log/sigmoid (lib.rs:768-932, 1154-1178)."""
    _need_f32(x)
    y = torch.empty_like(x)
    _ffi.call("hx_unary_f32", UNARY[op], x.numel(), _p(x), float(scalar), _p(y), None)
    return y


def mean(x: torch.Tensor, dims=None) -> torch.Tensor:
    """TensorReduce::mean (lib.rs:995-1010): each listed axis (all when None) removed in reverse
    list order by ndarray's mean_axis, with ndarray's summation order (bit-exact)."""
    _need_f32(x)
    order = list(range(x.dim())) if dims is None else list(dims)
    cur = x
    for ax in reversed(order):
        d = list(cur.shape)
        if ax >= len(d) or d[ax] == 0:
            raise InvalidDimension(f"Invalid dimension: {ax} is out of bounds for shape {d}")
        outer = 1
        for v in d[:ax]:
            outer *= v
        inner = 1
        for v in d[ax + 1:]:
            inner *= v
        y = torch.empty(d[:ax] + d[ax + 1:], device=x.device, dtype=torch.float32)
        _ffi.call("hx_mean_axis_f32", outer, d[ax], inner, 1 if ax == len(d) - 1 else 0,
                  _p(cur), _p(y), None)
        cur = y
    return cur if order else x.clone()


def _strides(dims):
    s = [1] * len(dims)
    for i in range(len(dims) - 1, 0, -1):
        s[i - 1] = s[i] * dims[i]
    return s


def copy_strided(shape, src: torch.Tensor, src_strides, dst: torch.Tensor, dst_strides,
                 src_offset: int = 0, dst_offset: int = 0) -> None:
    """dst[offset + sum c_j * dst_strides[j]] = src[offset + sum c_j * src_strides[j]] (elements)."""
    n = len(shape)
    if n > MAX_DIMS:
        raise UnsupportedOperation("more than 8 dimensions")
    arr = ctypes.c_int64 * max(n, 1)
    sp = ctypes.c_void_p(src.data_ptr() + 4 * src_offset)
    dp = ctypes.c_void_p(dst.data_ptr() + 4 * dst_offset)
    _ffi.call("hx_copy_strided_f32", n, arr(*shape), sp, arr(*src_strides), dp, arr(*dst_strides), None)


def broadcast_to(x: torch.Tensor, shape) -> torch.Tensor:
    """TensorBroadcast::broadcast_to (lib.rs:1352-1518; generic index map lib.rs:511-560 as
    written, quirk included)."""
    _need_f32(x)
    s, t = list(x.shape), list(shape)
    if len(s) > len(t):
        raise ShapeMismatch(f"Shape mismatch: expected [{len(t)}], got [{len(s)}]")
    if s == t:
        return x.clone()
    padded = [1] * (len(t) - len(s)) + s
    for pd, td in zip(padded, t):
        if pd != 1 and pd != td:
            raise ShapeMismatch(f"Shape mismatch: expected [{td}], got [{pd}]")
    if (len(s), len(t)) == (1, 2):
        if s[0] == t[1]:
            src = [0, 1]
        elif s[0] == t[0]:
            src = [1, 0]
        else:
            raise ShapeMismatch(f"Shape mismatch: expected [{t[1]}], got [{s[0]}]")
    elif (len(s), len(t)) == (2, 3):
        if s == t[1:]:
            src = [0, s[1], 1]
        elif s[0] == 1 and s[1] == t[2]:
            src = [0, 0, 1]
        else:
            raise ShapeMismatch(f"Shape mismatch: expected {t[1:]}, got {s}")
    elif (len(s), len(t)) == (1, 3):
        if s[0] != t[2]:
            raise ShapeMismatch(f"Shape mismatch: expected [{t[2]}], got [{s[0]}]")
        src = [0, 0, 1]
    else:
        if not s:
            raise InvalidDimension("Invalid dimension: 0 is out of bounds for shape []")
        ss = _strides(s)
        src = [(ss[j] if j < len(ss) else 1) if padded[j] != 1 else 0 for j in range(len(t))]
    y = torch.empty(t, device=x.device, dtype=torch.float32)
    if y.numel():
        copy_strided(t, x, src, y, _strides(t))
    return y


def transpose(x: torch.Tensor, d0: int, d1: int) -> torch.Tensor:
    """Tensor::transpose (lib.rs:115-137), materialised row-major."""
    _need_f32(x)
    s = list(x.shape)
    if d0 >= len(s) or d1 >= len(s):
        raise InvalidDimension(f"Invalid dimension: {max(d0, d1)} is out of bounds for shape {s}")
    nd = list(s)
    nd[d0], nd[d1] = nd[d1], nd[d0]
    src = _strides(s)
    src[d0], src[d1] = src[d1], src[d0]
    y = torch.empty(nd, device=x.device, dtype=torch.float32)
    if y.numel():
        copy_strided(nd, x, src, y, _strides(nd))
    return y


def slice(x: torch.Tensor, start, end) -> torch.Tensor:  # noqa: A001 - the reference's name
    """Tensor::slice (lib.rs:139-183): 2-D only, the reference's bounds errors."""
    s = list(x.shape)
    if len(start) != len(s) or len(end) != len(s):
        raise ShapeMismatch(f"Shape mismatch: expected [{len(s)}], got [{max(len(start), len(end))}]")
    for i, (a, b) in enumerate(zip(start, end)):
        if a >= s[i] or b > s[i] or a >= b:
            raise InvalidDimension(f"Invalid dimension: {i} is out of bounds for shape {s}")
    if len(s) != 2:
        raise UnsupportedOperation(f"Slicing for {len(s)}D tensors not implemented yet")
    _need_f32(x)
    nd = [end[0] - start[0], end[1] - start[1]]
    y = torch.empty(nd, device=x.device, dtype=torch.float32)
    copy_strided(nd, x, [s[1], 1], y, [nd[1], 1], src_offset=start[0] * s[1] + start[1])
    return y


def stack(tensors, dim: int):
    """Tensor::stack (lib.rs:254-335, 390-467): returns (data tensor, the reference's shape field).
    1..3-D inputs: data back to back whatever `dim`; others: a true stack along `dim`."""
    if not tensors:
        raise UnsupportedOperation("stacking of empty tensor list")
    if len(tensors) == 1:
        return tensors[0].clone(), list(tensors[0].shape)
    f = list(tensors[0].shape)
    for t in tensors[1:]:
        if list(t.shape) != f:
            raise ShapeMismatch(f"Shape mismatch: expected {f}, got {list(t.shape)}")
    if dim > len(f):
        raise InvalidDimension(f"Invalid dimension: {dim} is out of bounds for shape {f}")
    field = f[:dim] + [len(tensors)] + f[dim:]
    y = torch.empty(field, device=tensors[0].device, dtype=torch.float32)
    each = tensors[0].numel()
    if 1 <= len(f) <= 3:
        for k, t in enumerate(tensors):
            _need_f32(t)
            if each:
                copy_strided([each], t, [1], y, [1], dst_offset=k * each)
        return y, field
    if not f:
        raise InvalidDimension("Invalid dimension: 0 is out of bounds for shape []")
    outer = 1
    for v in f[:dim]:
        outer *= v
    inner = 1
    for v in f[dim:]:
        inner *= v
    for k, t in enumerate(tensors):
        _need_f32(t)
        if each:
            copy_strided([outer, inner], t, [inner, 1], y, [len(tensors) * inner, 1],
                         dst_offset=k * inner)
    return y, field


def cat(tensors, dim: int) -> torch.Tensor:
    """Tensor::cat (lib.rs:185-252): 1-D only beyond the reference's shape checks."""
    if not tensors:
        raise UnsupportedOperation("concatenation of empty tensor list")
    if len(tensors) == 1:
        return tensors[0].clone()
    f = list(tensors[0].shape)
    if dim >= len(f):
        raise InvalidDimension(f"Invalid dimension: {dim} is out of bounds for shape {f}")
    for t in tensors[1:]:
        o = list(t.shape)
        if len(o) != len(f):
            raise ShapeMismatch(f"Shape mismatch: expected [{len(f)}], got [{len(o)}]")
        for i, (a, b) in enumerate(zip(f, o)):
            if i != dim and a != b:
                raise ShapeMismatch(f"Shape mismatch: expected [{a}], got [{b}]")
    if len(f) != 1:
        raise UnsupportedOperation(f"Concatenation for {len(f)}D tensors not implemented yet")
    total = sum(t.numel() for t in tensors)
    y = torch.empty(total, device=tensors[0].device, dtype=torch.float32)
    off = 0
    for t in tensors:
        _need_f32(t)
        if t.numel():
            copy_strided([t.numel()], t, [1], y, [1], dst_offset=off)
        off += t.numel()
    return y


def fill(shape, value: float, device) -> torch.Tensor:
    """Tensor zeros / ones / from_scalar (lib.rs:1273-1301, 904-914)."""
    y = torch.empty(list(shape), device=device, dtype=torch.float32)
    _ffi.call("hx_fill_f32", y.numel(), float(value), _p(y), None)
    return y


def eye(n: int, device) -> torch.Tensor:
    """TensorRandom::eye (lib.rs:1303-1323)."""
    y = torch.empty((n, n), device=device, dtype=torch.float32)
    _ffi.call("hx_eye_f32", n, _p(y), None)
    return y
