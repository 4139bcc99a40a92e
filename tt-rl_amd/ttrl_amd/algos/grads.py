"""Gradient-norm measurement and clipping (ttrl/algos/grads.py:13-60)."""

from __future__ import annotations

import numpy as np

from ttrl_amd.engine.autograd import Tensor
from ttrl_amd.engine.ops import _kernels as K
from ttrl_amd.engine.pending import settle
from ttrl_amd.engine.tensor import arena_of, zeros

__all__ = ["clip_grad_norm", "grad_norm", "grad_sq_device", "param_snapshot"]


def grad_norm(params) -> float:
    """Global L2 norm (float64 on the host) over parameters holding a gradient."""
    params = list(params)
    settle(params)
    total = 0.0
    for p in params:
        if p.grad is None:
            continue
        arr = p.grad.numpy().astype(np.float64)
        total += float(np.sum(arr * arr))
    return float(np.sqrt(total))


def clip_grad_norm(params, max_norm: float) -> float:
    """Scale every gradient so the global norm is at most max_norm; returns the norm before."""
    if not max_norm > 0.0:
        raise ValueError(f"clip_grad_norm: max_norm must be > 0, got {max_norm}")
    params = list(params)
    total = grad_norm(params)
    if total > max_norm:
        scale = max_norm / (total + 1e-6)
        for p in params:
            if p.grad is not None:
                buf, _ = p._grad_target()
                K.unary("mul_s", buf, scale, out=buf)
    return total


def grad_sq_device(params):
    """Sum of squared gradients as a (1, 1) device array, or None without gradients.

    Over a whole arena whose gradient slots hold every gradient this is one
    reduction of the flat gradient buffer."""
    params = list(params)
    settle(params)
    have = [p for p in params if p.grad is not None]
    if not have:
        return None
    dev = have[0].device
    out = zeros(dev, (1, 1))
    arena = arena_of(params)
    if arena is not None and len(have) == len(params) and all(p.grad is p._grad_slot for p in params):
        dev.call("ttrl_sum_squares", arena.grad.vp, arena.numel, out.vp, 0)
        return out
    first = True
    for p in have:
        dev.call("ttrl_sum_squares", p.grad.vp, p.grad.numel, out.vp, int(not first))
        first = False
    return out


def param_snapshot(module) -> dict[str, np.ndarray]:
    return {name: p.numpy().copy() for name, p in module.named_parameters()}
