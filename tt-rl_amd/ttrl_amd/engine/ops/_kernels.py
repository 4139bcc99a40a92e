"""Array-level launchers over libttrl_hip for the primitive ops.

Every function takes and returns `DeviceArray`s and only enqueues kernels on
the device's stream (no host reads), so any composition of them can be
captured into a graph.
"""

from __future__ import annotations

import ctypes as C

import numpy as np

from ttrl_amd import _lib
from ttrl_amd.engine.tensor import DeviceArray

F32 = np.float32


def _contig_strides(shape) -> list[int]:
    strides, acc = [], 1
    for d in reversed(shape):
        strides.append(acc)
        acc *= int(d)
    return list(reversed(strides))


def broadcast_shape(a, b) -> tuple[int, ...]:
    try:
        return tuple(int(d) for d in np.broadcast_shapes(tuple(a), tuple(b)))
    except ValueError as e:
        raise ValueError(f"shapes {tuple(a)} and {tuple(b)} do not broadcast") from e


def _bstrides(shape, out_shape) -> list[int]:
    """Element strides of a contiguous `shape` read as `out_shape` (0 = broadcast)."""
    pad = len(out_shape) - len(shape)
    full = (1,) * pad + tuple(shape)
    base = _contig_strides(full)
    return [0 if full[i] == 1 and out_shape[i] != 1 else base[i] for i in range(len(out_shape))]


def _need_f32(*arrays):
    for a in arrays:
        if a.dtype != F32:
            raise ValueError(f"op expects float32 device data, got {a.dtype}")


def unary(op: str, a: DeviceArray, scalar: float = 0.0, out: DeviceArray | None = None) -> DeviceArray:
    _need_f32(a)
    y = out if out is not None else DeviceArray(a.dev, a.shape)
    a.dev.call("ttrl_unary", _lib.U[op], a.vp, y.vp, C.c_long(a.numel), C.c_float(scalar))
    return y


def binary_into(op: str, a: DeviceArray, b: DeviceArray, y: DeviceArray) -> DeviceArray:
    _need_f32(a, b, y)
    shape = broadcast_shape(a.shape, b.shape)
    if tuple(y.shape) != shape:
        raise ValueError(f"binary_into: output {y.shape} is not the broadcast shape {shape}")
    nd = max(1, len(shape))
    sh = shape if shape else (1,)
    sa = _bstrides(a.shape if a.shape else (1,), sh)
    sb = _bstrides(b.shape if b.shape else (1,), sh)
    a.dev.call("ttrl_binary", _lib.BOP[op], a.vp, b.vp, y.vp, nd, _lib.longs(sh), _lib.longs(sa), _lib.longs(sb))
    return y


def binary(op: str, a: DeviceArray, b: DeviceArray) -> DeviceArray:
    shape = broadcast_shape(a.shape, b.shape)
    return binary_into(op, a, b, DeviceArray(a.dev, shape))


def full_like(a: DeviceArray, value: float) -> DeviceArray:
    y = DeviceArray(a.dev, a.shape)
    y.fill(value)
    return y


def reduce_dim(op: str, a: DeviceArray, dim: int, keepdim: bool = True) -> DeviceArray:
    _need_f32(a)
    rank = len(a.shape)
    d = dim if dim >= 0 else dim + rank
    if not 0 <= d < rank:
        raise ValueError(f"reduce: dim {dim} out of range for shape {a.shape}")
    outer = int(np.prod(a.shape[:d], dtype=np.int64)) if d else 1
    inner = int(np.prod(a.shape[d + 1:], dtype=np.int64)) if d + 1 < rank else 1
    n = int(a.shape[d])
    out_shape = tuple(a.shape[:d]) + ((1,) if keepdim else ()) + tuple(a.shape[d + 1:])
    y = DeviceArray(a.dev, out_shape)
    a.dev.call("ttrl_reduce", _lib.R[op], a.vp, y.vp, C.c_long(outer), C.c_long(n), C.c_long(inner))
    return y


def sum_all(a: DeviceArray) -> DeviceArray:
    _need_f32(a)
    y = DeviceArray(a.dev, (1,) * max(1, len(a.shape)))
    a.dev.call("ttrl_reduce", _lib.R["sum"], a.vp, y.vp, C.c_long(1), C.c_long(a.numel), C.c_long(1))
    return y


def copy_region(src: DeviceArray, src_begin, dst: DeviceArray, dst_begin, extent) -> None:
    """dst[dst_begin + i] = src[src_begin + i] over an `extent` box."""
    rank = len(extent)
    ss = _contig_strides(src.shape)
    ds = _contig_strides(dst.shape)
    src_off = sum(int(b) * s for b, s in zip(src_begin, ss))
    dst_off = sum(int(b) * s for b, s in zip(dst_begin, ds))
    if any(int(e) == 0 for e in extent):
        return
    a = src.view(src_off, (src.numel - src_off,))
    y = dst.view(dst_off, (dst.numel - dst_off,))
    src.dev.call("ttrl_copy_strided", a.vp, y.vp, rank, _lib.longs(extent), _lib.longs(ss), _lib.longs(ds))


def repeat_to(a: DeviceArray, shape) -> DeviceArray:
    """Broadcast-expand `a` (equal rank, axes 1 or equal) to `shape`."""
    y = DeviceArray(a.dev, shape)
    sa = _bstrides(a.shape, tuple(shape))
    a.dev.call("ttrl_copy_strided", a.vp, y.vp, len(shape), _lib.longs(shape), _lib.longs(sa),
               _lib.longs(_contig_strides(shape)))
    return y


def matmul_raw(a: DeviceArray, b: DeviceArray, *, ta=False, tb=False, out=None, beta=0.0) -> DeviceArray:
    """Rank-2 product op(a) @ op(b) on the MFMA core."""
    _need_f32(a, b)
    if len(a.shape) != 2 or len(b.shape) != 2:
        raise ValueError("matmul_raw: rank-2 operands only")
    M, K = (a.shape[1], a.shape[0]) if ta else a.shape
    K2, N = (b.shape[1], b.shape[0]) if tb else b.shape
    if K != K2:
        raise ValueError(f"matmul: inner dims differ ({a.shape}{'T' if ta else ''} @ {b.shape}{'T' if tb else ''})")
    y = out if out is not None else DeviceArray(a.dev, (M, N))
    a.dev.call("ttrl_matmul", int(M), int(N), int(K), a.vp, C.c_long(a.shape[1]), int(ta), b.vp,
               C.c_long(b.shape[1]), int(tb), y.vp, C.c_long(N), C.c_float(1.0), C.c_float(beta))
    return y
