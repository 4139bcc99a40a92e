"""Gradient shape plumbing for broadcasting ops (the bias-gradient reduction
of ttrl/engine/ops/broadcast.py:11-30 and the sum backward's expansion of
:33-54).

`sum_to_shape` folds a gradient back onto an operand that was broadcast.
The operand's shape is right-aligned against the gradient's; every gradient
axis the operand did not have, or had with extent 1, is summed.  Consecutive
summed axes form one run, and each run is one `ttrl_reduce` launch over the
[outer][run][inner] view of the buffer, so a bias gradient [B, N] -> [N] or a
conv bias gradient [1, 1, P, C] -> [1, 1, 1, C] is a single launch whatever
the rank.

`expand_to` is the inverse direction: a keepdim-shaped gradient of a
reduction repeated back over the reduced axes.
"""

from __future__ import annotations

import math

from ttrl_amd.engine.ops import _kernels as K

__all__ = ["sum_to_shape", "expand_to"]


def _summed_runs(grad_shape, target_shape):
    """[(first_axis, last_axis)] of maximal runs of gradient axes to sum."""
    lead = len(grad_shape) - len(target_shape)
    if lead < 0:
        raise ValueError(f"a gradient of shape {tuple(grad_shape)} has fewer axes than the operand "
                         f"{tuple(target_shape)} it flows into")
    runs, start = [], None
    for axis, extent in enumerate(grad_shape):
        t = 1 if axis < lead else int(target_shape[axis - lead])
        summed = t == 1 and int(extent) != 1
        if not summed and t != int(extent):
            raise ValueError(f"gradient axis {axis} of extent {extent} cannot fold onto operand extent {t} "
                             f"(gradient {tuple(grad_shape)}, operand {tuple(target_shape)})")
        if summed and start is None:
            start = axis
        elif not summed and start is not None:
            runs.append((start, axis - 1))
            start = None
    if start is not None:
        runs.append((start, len(grad_shape) - 1))
    return runs


def sum_to_shape(grad, target_shape):
    """Sum `grad` (a DeviceArray) onto `target_shape`, one launch per run of
    broadcast axes; returns an array of exactly `target_shape`."""
    target_shape = tuple(int(d) for d in target_shape)
    shape = [int(d) for d in grad.shape]
    if tuple(shape) == target_shape:
        return grad
    for first, last in reversed(_summed_runs(shape, target_shape)):
        outer = math.prod(shape[:first])
        run = math.prod(shape[first:last + 1])
        inner = math.prod(shape[last + 1:])
        grad = K.reduce_dim("sum", grad.reshape((outer, run, inner)), 1, keepdim=True)
        shape = shape[:first] + [1] * (last + 1 - first) + shape[last + 1:]
        grad = grad.reshape(shape)
    return grad.reshape(target_shape)


def expand_to(grad, shape):
    """Repeat a keepdim-shaped gradient over the axes where it has extent 1
    and `shape` does not (the backward of a sum); other axes must agree."""
    shape = tuple(int(d) for d in shape)
    have = tuple(int(d) for d in grad.shape)
    if len(have) != len(shape):
        raise ValueError(f"expand_to: gradient rank {len(have)} differs from the target rank {len(shape)}; "
                         "keep the reduced axes (keepdim) before expanding")
    bad = [ax for ax, (g, t) in enumerate(zip(have, shape)) if g != t and g != 1]
    if bad:
        raise ValueError(f"expand_to: gradient {have} cannot expand to {shape}: axes {bad} are neither equal "
                         "nor of extent 1")
    return grad if have == shape else K.repeat_to(grad, shape)
