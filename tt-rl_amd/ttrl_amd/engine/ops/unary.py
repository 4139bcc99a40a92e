"""Unary elementwise ops with their closed-form backward
(ttrl/engine/ops/unary.py:21-150): exp, tanh, sigmoid reuse the saved output,
log and sqrt divide, relu masks on the input (relu_bw is 0 at 0)."""

from __future__ import annotations

from ttrl_amd.engine.autograd import Tensor, _detached, _needs
from ttrl_amd.engine.ops import _kernels as K
from ttrl_amd.engine.ops.elementwise import mul


def neg(a: Tensor) -> Tensor:
    return mul(a, -1.0)


def _unary(a: Tensor, op: str, name: str, backward):
    y = K.unary(op, a.data)
    if not _needs(a):
        return _detached(y)
    out = Tensor(y, True, (a,), name)
    x = a.data

    def _backward(grad):
        if a.requires_grad:
            a._accumulate(backward(grad, x, y))

    out._backward = _backward
    return out


def relu(a: Tensor) -> Tensor:
    return _unary(a, "relu", "relu", lambda g, x, y: K.binary("relu_bw", g, x))


def abs_(a: Tensor) -> Tensor:
    return _unary(a, "abs", "abs", lambda g, x, y: K.binary("mul", g, K.unary("sign", x)))


def square(a: Tensor) -> Tensor:
    return _unary(a, "square", "square", lambda g, x, y: K.binary("mul", g, K.unary("mul_s", x, 2.0)))


def exp(a: Tensor) -> Tensor:
    return _unary(a, "exp", "exp", lambda g, x, y: K.binary("mul", g, y))


def log(a: Tensor) -> Tensor:
    """Natural log; input must be > 0."""
    return _unary(a, "log", "log", lambda g, x, y: K.binary("div", g, x))


def tanh(a: Tensor) -> Tensor:
    return _unary(a, "tanh", "tanh",
                  lambda g, x, y: K.binary("mul", g, K.unary("rsub_s", K.binary("mul", y, y), 1.0)))


def sigmoid(a: Tensor) -> Tensor:
    return _unary(a, "sigmoid", "sigmoid",
                  lambda g, x, y: K.binary("mul", g, K.binary("mul", y, K.unary("rsub_s", y, 1.0))))


def sqrt(a: Tensor) -> Tensor:
    """Square root; input must be > 0 (the derivative is unbounded at 0)."""
    return _unary(a, "sqrt", "sqrt", lambda g, x, y: K.binary("div", g, K.unary("mul_s", y, 2.0)))
