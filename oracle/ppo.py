"""Numpy restatement of PPO's per-rollout and per-minibatch arithmetic.

gae                  float32 recursion exactly as ttrl/buffers/rollout.py:195-226
                     (t = T-1 .. 0; delta = r + gamma*V'*(1-d) - V;
                     A = delta + gamma*lam*(1-d)*A'; A *= valid; R = A + V),
                     with the reference's rounding: float32 arrays times Python
                     floats (gamma rounded to float32, gamma*lam formed in
                     double then rounded)
normalize_advantages (a - mean) / (std + 1e-8) over valid entries,
                     ttrl/buffers/rollout.py:269-270 (population std)
log_softmax/entropy  ttrl/engine/ops/functional.py:160-178 (detached max shift)
ppo_objective        ttrl/algos/ppo/loss.py:27-83 with the categorical head's
                     log-prob and entropy (ttrl/algos/ppo/policy.py:64-76);
                     minimum / maximum / clamp as the relu identities of
                     ttrl/engine/ops/select.py:39-63, whose gradients route a
                     tie to the first operand and vanish at clamp bounds
clip_grad_norm       ttrl/algos/grads.py:13-43 (float64 norm, scale
                     max_norm / (norm + 1e-6) when norm > max_norm)

Forward values and the analytic gradients d loss / d logits, d loss / d
values are float64.  Test infrastructure only.
"""

from __future__ import annotations

import numpy as np


def gae(rewards, values, dones, last_values, gamma: float, lam: float, valid=None):
    """-> (advantages, returns), float32 [T][N]."""
    rewards = np.asarray(rewards, np.float32)
    values = np.asarray(values, np.float32)
    dones = np.asarray(dones, np.float32)
    T, N = rewards.shape
    valid = np.ones((T, N), np.float32) if valid is None else np.asarray(valid, np.float32)
    g32 = np.float32(gamma)
    gl32 = np.float32(float(gamma) * float(lam))
    adv = np.zeros((T, N), np.float32)
    last_gae = np.zeros(N, np.float32)
    next_values = np.asarray(last_values, np.float32).reshape(N)
    for t in range(T - 1, -1, -1):
        not_done = np.float32(1.0) - dones[t]
        delta = (rewards[t] + (g32 * next_values) * not_done) - values[t]
        last_gae = delta + (gl32 * not_done) * last_gae
        last_gae = last_gae * valid[t]
        adv[t] = last_gae
        next_values = values[t]
    return adv, adv + values


def normalize_advantages(adv, valid=None, eps: float = 1e-8):
    """(a - mean) / (std + eps) over entries with valid > 0; 0 elsewhere."""
    a = np.asarray(adv, np.float64).reshape(-1)
    keep = np.ones(a.shape, bool) if valid is None else np.asarray(valid).reshape(-1) > 0
    mean = a[keep].mean()
    std = a[keep].std()
    out = np.where(keep, (a - mean) / (std + eps), 0.0)
    return out.reshape(np.shape(adv)), float(mean), float(std)


def log_softmax(z):
    z = np.asarray(z, np.float64)
    shifted = z - z.max(axis=-1, keepdims=True)
    return shifted - np.log(np.exp(shifted).sum(axis=-1, keepdims=True))


def entropy(z):
    lp = log_softmax(z)
    return -(np.exp(lp) * lp).sum(axis=-1)


def ppo_objective(logits, actions, old_logp, advantages, returns, old_values, values, valid=None, *,
                  clip_eps: float, value_clip_eps: float, value_coef: float, entropy_coef: float):
    """-> dict(loss, policy_loss, value_loss, entropy, new_logp[B], dlogits[B][A], dvalues[B])."""
    z = np.asarray(logits, np.float64)
    B, A = z.shape
    a = np.asarray(actions).reshape(-1).astype(np.int64)
    w = np.ones(B) if valid is None else np.asarray(valid, np.float64).reshape(-1)
    total = w.sum()
    lp_all = log_softmax(z)
    p = np.exp(lp_all)
    inside = (a >= 0) & (a < A)
    onehot = np.zeros((B, A))
    onehot[np.flatnonzero(inside), a[inside]] = 1.0
    lp = (lp_all * onehot).sum(axis=1)
    H = -(p * lp_all).sum(axis=1)

    ratio = np.exp(lp - np.asarray(old_logp, np.float64).reshape(-1))
    adv = np.asarray(advantages, np.float64).reshape(-1)
    lo, hi = 1.0 - clip_eps, 1.0 + clip_eps
    rc = np.minimum(np.maximum(ratio, lo), hi)
    u, c = ratio * adv, rc * adv
    surr = u - np.maximum(u - c, 0.0)
    take_u = ~(u - c > 0.0)
    dclamp = ((ratio > lo) & (ratio < hi)).astype(np.float64)
    dsurr_dr = np.where(take_u, adv, dclamp * adv)
    policy_loss = -(surr * w).sum() / total

    v = np.asarray(values, np.float64).reshape(-1)
    ov = np.asarray(old_values, np.float64).reshape(-1)
    R = np.asarray(returns, np.float64).reshape(-1)
    dv = v - ov
    dvc = np.minimum(np.maximum(dv, -value_clip_eps), value_clip_eps)
    eu, ec = v - R, (ov + dvc) - R
    qu, qc = eu * eu, ec * ec
    take_c = qc - qu > 0.0
    vmax = np.where(take_c, qc, qu)
    dvclamp = ((dv > -value_clip_eps) & (dv < value_clip_eps)).astype(np.float64)
    dq_dv = np.where(take_c, 2.0 * ec * dvclamp, 2.0 * eu)
    value_loss = 0.5 * (vmax * w).sum() / total
    ent = (H * w).sum() / total
    loss = policy_loss + value_coef * value_loss - entropy_coef * ent

    gp = np.where(inside, -w / total * dsurr_dr * ratio, 0.0)
    dlogits = gp[:, None] * (onehot - p) + (entropy_coef * w / total)[:, None] * p * (lp_all + H[:, None])
    dvalues = value_coef * 0.5 * w / total * dq_dv
    return dict(loss=loss, policy_loss=policy_loss, value_loss=value_loss, entropy=ent, new_logp=lp,
                dlogits=dlogits, dvalues=dvalues)


def clip_grad_norm(g, max_norm: float):
    """-> (clipped float32 gradient, norm before clipping)."""
    g = np.asarray(g, np.float32)
    total = float(np.sqrt(np.sum(g.astype(np.float64) ** 2)))
    if total > max_norm:
        g = g * np.float32(max_norm / (total + 1e-6))
    return g, total
