"""Adam, restated two ways.

fused     the stored-S/V form with folded bias correction
          (ttrl/engine/optim/adam.py:93-134, ttrl/engine/optim/scalars.py:13-27)
textbook  m/v with explicit bias correction (tests/engine/test_optim.py:27-44
          in the reference), used to pin the fused form.
"""

from __future__ import annotations

import math

import numpy as np

from oracle import fa, float_type


def fused_scalars(lr, b1, b2, eps, t):
    if t < 1:
        raise ValueError("t must be >= 1")
    bc1 = 1 - b1 ** t
    bc2 = 1 - b2 ** t
    c = math.sqrt((1 - b2) / bc2)
    return lr * (1 - b1) / bc1 / c, eps / c


def fused_step(p, g, S, V, t, lr, b1=0.9, b2=0.999, eps=1e-8, weight_decay=0.0):
    """One update in the stored form; returns (p, S, V) as float64."""
    p = fa(p)
    g = fa(g)
    if weight_decay:
        g = g + weight_decay * p
    V = g * g + b2 * fa(V)
    S = g + b1 * fa(S)
    alpha_t, eps_t = fused_scalars(lr, b1, b2, eps, t)
    return p - alpha_t * S / (np.sqrt(V) + eps_t), S, V


def textbook_step(p, g, m, v, t, lr, b1=0.9, b2=0.999, eps=1e-8):
    p = fa(p)
    g = fa(g)
    m = b1 * fa(m) + (1 - b1) * g
    v = b2 * fa(v) + (1 - b2) * g * g
    mhat = m / (1 - b1 ** t)
    vhat = v / (1 - b2 ** t)
    return p - lr * mhat / (np.sqrt(vhat) + eps), m, v
