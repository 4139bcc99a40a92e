"""Broadcast-gradient reduction and expansion (ttrl/engine/ops/broadcast.py:11-54)."""

from __future__ import annotations

from ttrl_amd.engine.ops import _kernels as K


def _reduce_broadcast_grad(grad, target_shape):
    """Sum `grad` back down to `target_shape` along every broadcast dim."""
    grad_shape = tuple(grad.shape)
    target_shape = tuple(target_shape)
    pad = len(grad_shape) - len(target_shape)
    assert pad >= 0, "grad rank must be >= operand rank"
    padded_target = (1,) * pad + target_shape
    for dim, (g_sz, t_sz) in enumerate(zip(grad_shape, padded_target)):
        if t_sz == 1 and g_sz != 1:
            grad = K.reduce_dim("sum", grad, dim, keepdim=True)
    if pad:
        grad = grad.reshape(target_shape)
    return grad


def _broadcast_grad_to(grad, like):
    """Expand a reduced gradient back to `like`'s shape."""
    gshape = tuple(int(d) for d in grad.shape)
    tshape = tuple(int(d) for d in like.shape)
    if len(gshape) != len(tshape):
        raise ValueError(
            f"cannot broadcast gradient of rank {len(gshape)} back to rank "
            f"{len(tshape)}: reshape it to a keepdim shape first."
        )
    for g, t in zip(gshape, tshape):
        if g != t and g != 1:
            raise ValueError(
                f"cannot broadcast gradient of shape {gshape} back to {tshape}: "
                "axis sizes must be equal or 1."
            )
    if gshape == tshape:
        return grad
    return K.repeat_to(grad, tshape)
