"""Binary elementwise arithmetic: add, sub, mul, div
(ttrl/engine/ops/elementwise.py:15-148).  A python-scalar operand goes to the
kernel as an argument; tensor operands broadcast, and the backward sums the
gradient back over every broadcast axis."""

from __future__ import annotations

from ttrl_amd.engine.autograd import Tensor, _detached, _is_scalar, _needs
from ttrl_amd.engine.ops import _kernels as K
from ttrl_amd.engine.ops.broadcast import _reduce_broadcast_grad


def _as_tensor(x, like: Tensor) -> Tensor:
    if isinstance(x, Tensor):
        return x
    return Tensor(K.full_like(like.data, float(x)), requires_grad=False)


def add(a: Tensor, b) -> Tensor:
    if _is_scalar(b):
        y = K.unary("add_s", a.data, float(b))
        if not _needs(a):
            return _detached(y)
        out = Tensor(y, True, (a,), "add")

        def _backward_scalar(grad):
            if a.requires_grad:
                a._accumulate(grad)

        out._backward = _backward_scalar
        return out
    b = _as_tensor(b, a)
    y = K.binary("add", a.data, b.data)
    if not _needs(a, b):
        return _detached(y)
    out = Tensor(y, True, (a, b), "add")

    def _backward(grad):
        if a.requires_grad:
            a._accumulate(_reduce_broadcast_grad(grad, a.shape))
        if b.requires_grad:
            b._accumulate(_reduce_broadcast_grad(grad, b.shape))

    out._backward = _backward
    return out


def sub(a, b) -> Tensor:
    if isinstance(a, Tensor) and _is_scalar(b):
        y = K.unary("add_s", a.data, -float(b))
        if not _needs(a):
            return _detached(y)
        out = Tensor(y, True, (a,), "sub")

        def _backward_scalar(grad):
            if a.requires_grad:
                a._accumulate(grad)

        out._backward = _backward_scalar
        return out
    if isinstance(b, Tensor) and _is_scalar(a):
        y = K.unary("rsub_s", b.data, float(a))
        if not _needs(b):
            return _detached(y)
        out = Tensor(y, True, (b,), "sub")

        def _backward_rscalar(grad):
            if b.requires_grad:
                b._accumulate(K.unary("neg", grad))

        out._backward = _backward_rscalar
        return out
    if not isinstance(a, Tensor) or not isinstance(b, Tensor):
        raise TypeError(f"sub expects Tensor operands or one scalar, got {type(a)} and {type(b)}")
    y = K.binary("sub", a.data, b.data)
    if not _needs(a, b):
        return _detached(y)
    out = Tensor(y, True, (a, b), "sub")

    def _backward(grad):
        if a.requires_grad:
            a._accumulate(_reduce_broadcast_grad(grad, a.shape))
        if b.requires_grad:
            b._accumulate(_reduce_broadcast_grad(K.unary("neg", grad), b.shape))

    out._backward = _backward
    return out


def mul(a: Tensor, b) -> Tensor:
    if _is_scalar(b):
        s = float(b)
        y = K.unary("mul_s", a.data, s)
        if not _needs(a):
            return _detached(y)
        out = Tensor(y, True, (a,), "mul")

        def _backward_scalar(grad):
            if a.requires_grad:
                a._accumulate(K.unary("mul_s", grad, s))

        out._backward = _backward_scalar
        return out
    b = _as_tensor(b, a)
    y = K.binary("mul", a.data, b.data)
    if not _needs(a, b):
        return _detached(y)
    out = Tensor(y, True, (a, b), "mul")
    a_data, b_data = a.data, b.data

    def _backward(grad):
        if a.requires_grad:
            a._accumulate(_reduce_broadcast_grad(K.binary("mul", grad, b_data), a.shape))
        if b.requires_grad:
            b._accumulate(_reduce_broadcast_grad(K.binary("mul", grad, a_data), b.shape))

    out._backward = _backward
    return out


def div(a: Tensor, b) -> Tensor:
    if _is_scalar(b):
        s = float(b)
        y = K.unary("div_s", a.data, s)
        if not _needs(a):
            return _detached(y)
        out = Tensor(y, True, (a,), "div")

        def _backward_scalar(grad):
            if a.requires_grad:
                a._accumulate(K.unary("div_s", grad, s))

        out._backward = _backward_scalar
        return out
    b = _as_tensor(b, a)
    y = K.binary("div", a.data, b.data)
    if not _needs(a, b):
        return _detached(y)
    out = Tensor(y, True, (a, b), "div")
    a_data, b_data = a.data, b.data

    def _backward(grad):
        if a.requires_grad:
            a._accumulate(_reduce_broadcast_grad(K.binary("div", grad, b_data), a.shape))
        if b.requires_grad:
            # d/db (a/b) = -a/b^2
            q = K.binary("div", a_data, K.binary("mul", b_data, b_data))
            gb = K.binary("mul", grad, K.unary("neg", q))
            b._accumulate(_reduce_broadcast_grad(gb, b.shape))

    out._backward = _backward
    return out
