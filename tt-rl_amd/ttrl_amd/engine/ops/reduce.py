"""Reductions and the detached max/argmax pair (ttrl/engine/ops/reduce.py:12-99)."""

from __future__ import annotations

from ttrl_amd.engine.autograd import Tensor, _detached, _needs
from ttrl_amd.engine.ops import _kernels as K
from ttrl_amd.engine.ops.broadcast import expand_to
from ttrl_amd.engine.ops.elementwise import mul


def sum_all(a: Tensor) -> Tensor:
    """Sum every element to a keepdim-shaped scalar."""
    y = K.sum_all(a.data)
    if not _needs(a):
        return _detached(y)
    out = Tensor(y, True, (a,), "sum_all")
    like = a.data

    def _backward(grad):
        if a.requires_grad:
            a._accumulate(expand_to(grad.reshape((1,) * len(like.shape)), like.shape))

    out._backward = _backward
    return out


def mean_all(a: Tensor) -> Tensor:
    n = 1
    for d in a.shape:
        n *= int(d)
    return mul(sum_all(a), 1.0 / n)


def sum_dim(a: Tensor, dim: int, keepdim: bool = True) -> Tensor:
    y = K.reduce_dim("sum", a.data, dim, keepdim)
    if not _needs(a):
        return _detached(y)
    out = Tensor(y, True, (a,), "sum_dim")
    like = a.data
    d = dim if dim >= 0 else dim + len(a.shape)

    def _backward(grad):
        if not a.requires_grad:
            return
        if not keepdim:
            grad = grad.reshape(tuple(like.shape[:d]) + (1,) + tuple(like.shape[d + 1:]))
        a._accumulate(expand_to(grad, like.shape))

    out._backward = _backward
    return out


def mean_dim(a: Tensor, dim: int, keepdim: bool = True) -> Tensor:
    d = dim if dim >= 0 else dim + len(a.shape)
    return mul(sum_dim(a, dim=dim, keepdim=keepdim), 1.0 / int(a.shape[d]))


def max_dim_detached(a: Tensor, dim: int, keepdim: bool = True) -> Tensor:
    """Max along one axis, deliberately not differentiable."""
    return Tensor(K.reduce_dim("max", a.data, dim, keepdim), requires_grad=False)


def argmax_dim_detached(a: Tensor, dim: int = -1, keepdim: bool = True) -> Tensor:
    """Index of the max (first index on ties) along one axis, as float32."""
    return Tensor(K.reduce_dim("argmax", a.data, dim, keepdim), requires_grad=False)
