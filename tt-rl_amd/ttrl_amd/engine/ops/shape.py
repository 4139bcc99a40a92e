"""concat, reshape and split (ttrl/engine/ops/shape.py:10-151)."""

from __future__ import annotations

from ttrl_amd.engine.autograd import Tensor, _detached, _needs
from ttrl_amd.engine.ops import _kernels as K
from ttrl_amd.engine.tensor import DeviceArray


def concat(tensors, dim: int = -1) -> Tensor:
    """Concatenate along `dim`; backward slices each operand's extent back out."""
    tensors = tuple(tensors)
    if not tensors:
        raise ValueError("concat needs at least one tensor")
    rank = len(tensors[0].shape)
    axis = dim if dim >= 0 else dim + rank
    for t in tensors:
        if len(t.shape) != rank:
            raise ValueError(f"concat operands must share a rank, got {[t.shape for t in tensors]}")
    out_shape = list(tensors[0].shape)
    out_shape[axis] = sum(int(t.shape[axis]) for t in tensors)
    y = DeviceArray(tensors[0].device, out_shape)
    offset = 0
    extents = []
    for t in tensors:
        begin = [0] * rank
        begin[axis] = offset
        K.copy_region(t.data, [0] * rank, y, begin, t.shape)
        extents.append(int(t.shape[axis]))
        offset += int(t.shape[axis])
    if not _needs(*tensors):
        return _detached(y)
    operands = tensors
    out = Tensor(y, True, operands, "concat")

    def _backward(grad):
        off = 0
        for operand, extent in zip(operands, extents):
            if operand.requires_grad:
                begin = [0] * rank
                begin[axis] = off
                piece = DeviceArray(grad.dev, operand.shape)
                K.copy_region(grad, begin, piece, [0] * rank, operand.shape)
                operand._accumulate(piece)
            off += extent

    out._backward = _backward
    return out


def reshape(a: Tensor, shape) -> Tensor:
    shape = tuple(int(d) for d in shape)
    in_shape = tuple(int(d) for d in a.shape)
    y = a.data.reshape(shape)
    if not _needs(a):
        return _detached(y)
    out = Tensor(y, True, (a,), "reshape")

    def _backward(grad):
        if a.requires_grad:
            a._accumulate(grad.reshape(in_shape), masked=out._grad_masked)

    out._backward = _backward
    return out


def split(a: Tensor, sizes, dim: int = -1) -> tuple[Tensor, ...]:
    """Cut `a` into consecutive pieces of `sizes` along `dim`."""
    sizes = tuple(int(s) for s in sizes)
    rank = len(a.shape)
    axis = dim if dim >= 0 else dim + rank
    if not 0 <= axis < rank:
        raise ValueError(
            f"split got dim={dim} for a rank-{rank} tensor of shape "
            f"{tuple(a.shape)}; dim must index an existing axis."
        )
    extent = int(a.shape[axis])
    if any(s <= 0 for s in sizes) or sum(sizes) != extent:
        raise ValueError(
            f"split sizes {sizes} must be positive and sum to {extent}, the "
            f"extent of axis {axis} in shape {tuple(a.shape)}; got sum {sum(sizes)}."
        )
    in_shape = tuple(int(d) for d in a.shape)
    pieces = []
    offset = 0
    for size in sizes:
        begin = [0] * rank
        begin[axis] = offset
        pshape = list(in_shape)
        pshape[axis] = size
        y = DeviceArray(a.device, pshape)
        K.copy_region(a.data, begin, y, [0] * rank, pshape)
        if not _needs(a):
            pieces.append(_detached(y))
        else:
            out = Tensor(y, True, (a,), "split")
            out._backward = _split_backward(a, in_shape, list(begin), pshape)
            pieces.append(out)
        offset += size
    return tuple(pieces)


def _split_backward(a: Tensor, in_shape, begin, pshape):
    def _backward(grad):
        if not a.requires_grad:
            return
        full = DeviceArray(grad.dev, in_shape)
        full.fill(0.0)
        K.copy_region(grad, [0] * len(in_shape), full, begin, pshape)
        a._accumulate(full)

    return _backward
