"""Tanh-squashed diagonal Gaussian in float64 (ttrl/algos/gaussian.py:55-117,
ttrl/algos/sac/policy.py:30-40): u = mean + exp(log_std)*eps, action =
centre + half_width*tanh(u), logp = sum(-z^2/2 - log_std) - d/2 log(2 pi)
- sum 2(log 2 - u - softplus(-2u)) - log_det, z = (u - mean)/exp(log_std)."""

from __future__ import annotations

import math

import numpy as np

from oracle import fa, float_type

LOG_2PI = math.log(2.0 * math.pi)
LOG_2 = math.log(2.0)


def softplus(x):
    return np.maximum(x, 0.0) + np.log1p(np.exp(-np.abs(x)))


def sample(mean, log_std, noise, centre=0.0, half_width=1.0, log_det=0.0):
    """-> (action, logp (B,), u)."""
    mean = fa(mean)
    log_std = fa(log_std)
    sigma = np.exp(log_std)
    u = mean + sigma * fa(noise)
    z = (u - mean) / sigma
    d = mean.shape[-1]
    normal = np.sum(-0.5 * z * z - log_std, axis=-1) - 0.5 * d * LOG_2PI
    corr = np.sum(2.0 * (LOG_2 - u - softplus(-2.0 * u)), axis=-1)
    logp = normal - corr - log_det
    return centre + half_width * np.tanh(u), logp, u


def sample_backward(mean, log_std, noise, g_action, g_logp, half_width=1.0):
    """dL/dmean, dL/dlog_std (before any clamp mask) for upstream
    dL/daction (B, d) and dL/dlogp (B,)."""
    mean = fa(mean)
    log_std = fa(log_std)
    sigma = np.exp(log_std)
    eps = fa(noise)
    u = mean + sigma * eps
    z = (u - mean) / sigma
    t = np.tanh(u)
    glp = fa(g_logp).reshape(-1, 1)
    gu = fa(g_action) * half_width * (1.0 - t * t) + glp * (2.0 * t - z / sigma)
    gmean = gu + glp * (z / sigma)
    gls = gu * sigma * eps + glp * (z * z - 1.0)
    return gmean, gls
