"""minimum / maximum / clamp through relu identities
(ttrl/engine/ops/select.py:39-63): the gradient routes to the selected side on
its own, min ties go to the first operand, and clamp's gradient is 1 strictly
inside (lo, hi) and 0 at and beyond the bounds."""

from __future__ import annotations

from ttrl_amd.engine.autograd import Tensor
from ttrl_amd.engine.ops.elementwise import add, sub
from ttrl_amd.engine.ops.unary import relu


def minimum(a: Tensor, b) -> Tensor:
    """min(a, b) = a - relu(a - b)."""
    return sub(a, relu(sub(a, b)))


def maximum(a: Tensor, b) -> Tensor:
    """max(a, b) = a + relu(b - a)."""
    return add(a, relu(sub(b, a)))


def clamp(x: Tensor, lo: float, hi: float) -> Tensor:
    """min(max(x, lo), hi) via two relu identities."""
    lifted_max = add(relu(sub(x, lo)), lo)
    return sub(hi, relu(sub(hi, lifted_max)))
