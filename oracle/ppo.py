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
minibatch_indices    RolloutBuffer.minibatches' shuffle (ttrl/buffers/rollout.py:239-282):
                     valid rows only, one rng.permutation per epoch, trailing
                     partial minibatch dropped
sequence_minibatches ttrl/buffers/seqbatch.py:40-120: whole sequences over
                     (chunk, lane), one permutation per epoch, rows
                     time-major (t * n_seq + sequence)
recurrent_ppo_step   ttrl/algos/ppo/recurrent.py:190-225 with
                     ttrl/nets/recurrent.py:49-196: trunk, ReLU, GRU unroll
                     from h0 with the episode-start mask, packed heads, the
                     objective's masked mean over valid slots, backward, clip,
                     Adam
ppo_update           ttrl/algos/ppo/learn.py:46-112 on a shared-trunk
                     actor-critic whose two heads are one Linear of width A+1
                     ([logits | value], ttrl/nets/models.py:65-71): GAE,
                     normalisation, then per minibatch forward, objective,
                     backward, clip_grad_norm, Adam (oracle.adam.fused_step),
                     approx_kl = mean(expm1(r) - r)

Forward values and the analytic gradients d loss / d logits, d loss / d
values are float64.  Test infrastructure only.
"""

from __future__ import annotations

import numpy as np

from oracle import adam
from oracle.gru import gru_backward, gru_forward
from oracle.nets import KINK_BAND, qnet_backward, qnet_forward


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


def minibatch_indices(valid, minibatch_size: int, epochs: int, rng) -> list:
    """Flat (time-major) row indices of every minibatch of one update."""
    keep = np.flatnonzero(np.asarray(valid).reshape(-1) > 0.0)
    total = int(keep.size)
    n_full = total // minibatch_size
    if n_full == 0:
        raise ValueError("minibatch_indices: fewer valid rows than one minibatch")
    out = []
    for _ in range(epochs):
        perm = rng.permutation(total)
        for start in range(0, n_full * minibatch_size, minibatch_size):
            out.append(keep[perm[start:start + minibatch_size]])
    return out


def ppo_minibatch_step(net, S: list, V: list, t: int, mb: dict, *, clip_eps: float = 0.1,
                       value_clip_eps: float = 0.1, value_coef: float = 0.5, entropy_coef: float = 0.01,
                       max_grad_norm: float = 0.5, lr: float = 2.5e-4, adam_eps: float = 1e-8,
                       betas=(0.9, 0.999), gates=None, stats=None) -> dict:
    """One minibatch step (ttrl/algos/ppo/learn.py:74-112) from parameters
    `net` and Adam state S, V (stored form) with update count t (>= 1).
    mb: obs, actions, old_logp, advantages, returns, values of the rows;
    gates: device ReLU gates adopted inside the kink band (oracle.nets.gate).
    -> dict(net, S, V, metrics, grads (clipped))."""
    out, acts = qnet_forward(net, mb["obs"], gates=gates, stats=stats)
    A = out.shape[1] - 1
    old_logp = np.asarray(mb["old_logp"], np.float64).reshape(-1)
    o = ppo_objective(out[:, :A], mb["actions"], old_logp, mb["advantages"], mb["returns"], mb["values"],
                      out[:, A], clip_eps=clip_eps, value_clip_eps=value_clip_eps, value_coef=value_coef,
                      entropy_coef=entropy_coef)
    dout = np.concatenate([o["dlogits"], o["dvalues"][:, None]], axis=1)
    grads = qnet_backward(net, acts, dout)
    norm = float(np.sqrt(sum(np.sum(g * g) for g in grads)))
    if norm > max_grad_norm:
        grads = [g * (max_grad_norm / (norm + 1e-6)) for g in grads]
    logratio = o["new_logp"] - old_logp
    params, S2, V2 = [], [], []
    for p, g, s_, v_ in zip(net.flat(), grads, S, V):
        p2, s2, v2 = adam.fused_step(p, g, s_, v_, t, lr, betas[0], betas[1], adam_eps)
        params.append(p2)
        S2.append(s2)
        V2.append(v2)
    metrics = dict(loss=o["loss"], policy_loss=o["policy_loss"], value_loss=o["value_loss"], entropy=o["entropy"],
                   approx_kl=float(np.mean(np.expm1(logratio) - logratio)), grad_norm=norm)
    return dict(net=net.with_flat(params), S=S2, V=V2, metrics=metrics, grads=grads)


def ppo_update(net, rollout: dict, *, rng, minibatch_size: int, epochs: int, gamma: float = 0.99,
               lam: float = 0.95, normalize_adv: bool = True, keep_grads: bool = False, **step_cfg) -> dict:
    """-> dict(net, steps=[per-step metrics], advantages, returns, batches[,
    grads]).  `net` is an oracle.nets.QNet whose last layer has A + 1
    outputs; batches[t] holds step t's minibatch rows, grads[t] its clipped
    gradients (with keep_grads); step_cfg goes to ppo_minibatch_step."""
    rewards = np.asarray(rollout["rewards"], np.float32)
    T, N = rewards.shape
    valid = rollout.get("valid")
    valid = np.ones((T, N), np.float32) if valid is None else np.asarray(valid, np.float32)
    adv, ret = gae(rewards, rollout["values"], rollout["dones"], rollout["last_values"], gamma, lam, valid)
    if normalize_adv:
        adv_n, _, _ = normalize_advantages(adv, valid)
    else:
        adv_n = adv.astype(np.float64)
    flat = dict(obs=np.asarray(rollout["obs"]).reshape((T * N,) + np.shape(rollout["obs"])[2:]),
                actions=np.asarray(rollout["actions"]).reshape(-1),
                old_logp=np.asarray(rollout["logp"], np.float64).reshape(-1),
                advantages=np.asarray(adv_n, np.float64).reshape(-1),
                returns=np.asarray(ret, np.float64).reshape(-1),
                values=np.asarray(rollout["values"], np.float64).reshape(-1))
    S = [np.zeros(np.shape(p)) for p in net.flat()]
    V = [np.zeros(np.shape(p)) for p in net.flat()]
    steps, kept, batches = [], [], []
    for t, idx in enumerate(minibatch_indices(valid, minibatch_size, epochs, rng), start=1):
        mb = {k: v[idx] for k, v in flat.items()}
        r = ppo_minibatch_step(net, S, V, t, mb, **step_cfg)
        net, S, V = r["net"], r["S"], r["V"]
        steps.append(r["metrics"])
        batches.append(mb)
        if keep_grads:
            kept.append(r["grads"])
    out = dict(net=net, steps=steps, advantages=adv, returns=ret, batches=batches)
    if keep_grads:
        out["grads"] = kept
    return out


def sequence_minibatches(T: int, N: int, seq_len: int, minibatch_size: int, epochs: int, rng) -> list:
    """-> [(rows (seq_len * n_seq,), h0 rows (n_seq,))] of flat time-major
    rollout indices (row t * N + lane) per minibatch, in the reference's
    shuffle order."""
    S = minibatch_size // seq_len
    total = (T // seq_len) * N
    n_full = total // S
    if n_full == 0:
        raise ValueError("sequence_minibatches: fewer sequences than one minibatch")
    out = []
    steps = np.arange(seq_len)
    for _ in range(epochs):
        perm = rng.permutation(total)
        for start in range(0, n_full * S, S):
            ids = perm[start:start + S]
            ch, ln = ids // N, ids % N
            rows = (ch[None, :] * seq_len + steps[:, None]) * N + ln[None, :]
            out.append((rows.reshape(-1), ch * N + ln))
    return out


def _relu_gate(z, gates, name):
    m = z > 0
    if gates is not None and name in gates:
        rms = np.sqrt(np.mean(z * z)) if z.size else 0.0
        near = np.abs(z) <= KINK_BAND * rms
        m = np.where(near, np.asarray(gates[name], bool).reshape(z.shape), m)
    return m.astype(np.float64)


def recurrent_ppo_step(params: dict, S: list, V: list, t: int, mb: dict, *, seq_len: int, clip_eps: float = 0.1,
                       value_clip_eps: float = 0.1, value_coef: float = 0.5, entropy_coef: float = 0.01,
                       max_grad_norm: float = 0.5, lr: float = 2.5e-4, adam_eps: float = 1e-8,
                       betas=(0.9, 0.999), gates=None) -> dict:
    """One recurrent minibatch step from parameters
    params = dict(trunk=QNet(convs, [fc1]), gru=(W_ih, W_hh, b_ih, b_hh),
    head=(W [H, A + 1], b)) and Adam state S, V (flat in the order trunk,
    gru, head) with update count t.  mb: obs, actions, old_logp, advantages,
    returns, values, valid (rows), starts (rows), h0 (n_seq, H).
    -> dict(params, S, V, metrics, grads)."""
    trunk, (W_ih, W_hh, b_ih, b_hh), (Wh, bh) = params["trunk"], params["gru"], params["head"]
    z1, acts = qnet_forward(trunk, mb["obs"], gates=gates)
    m1 = _relu_gate(z1, gates, "fc0")
    feat = z1 * m1
    rows, F = feat.shape
    n_seq = rows // seq_len
    H = W_hh.shape[0]
    starts = np.asarray(mb["starts"], np.float64).reshape(seq_len, n_seq)
    outs, cache = gru_forward(W_ih, W_hh, b_ih, b_hh, feat.reshape(seq_len, n_seq, F), mb["h0"], starts)
    state = outs.reshape(rows, H)
    out = state @ Wh + bh.reshape(1, -1)
    A = out.shape[1] - 1
    valid = np.asarray(mb["valid"], np.float64).reshape(-1)
    keep = valid > 0
    old_logp = np.where(keep, np.asarray(mb["old_logp"], np.float64).reshape(-1), 0.0)
    o = ppo_objective(out[:, :A], mb["actions"], old_logp, np.where(keep, mb["advantages"], 0.0),
                      np.where(keep, mb["returns"], 0.0), mb["values"], out[:, A], valid, clip_eps=clip_eps,
                      value_clip_eps=value_clip_eps, value_coef=value_coef, entropy_coef=entropy_coef)
    dout = np.concatenate([o["dlogits"], o["dvalues"][:, None]], axis=1)
    dWh, dbh = state.T @ dout, dout.sum(axis=0)
    dstate = dout @ Wh.T
    dseq, _dh0, dW_ih, dW_hh, db_ih, db_hh = gru_backward(cache, dstate.reshape(seq_len, n_seq, H))
    dfeat = dseq.reshape(rows, F) * m1
    grads = qnet_backward(trunk, acts, dfeat) + [dW_ih, dW_hh, db_ih, db_hh, dWh, dbh]
    norm = float(np.sqrt(sum(np.sum(g * g) for g in grads)))
    if norm > max_grad_norm:
        grads = [g * (max_grad_norm / (norm + 1e-6)) for g in grads]
    flat = trunk.flat() + [W_ih, W_hh, b_ih, b_hh, Wh, bh]
    new, S2, V2 = [], [], []
    for p, g, s_, v_ in zip(flat, grads, S, V):
        p2, s2, v2 = adam.fused_step(p, g, s_, v_, t, lr, betas[0], betas[1], adam_eps)
        new.append(p2)
        S2.append(s2)
        V2.append(v2)
    nt = len(trunk.flat())
    logratio = o["new_logp"] - old_logp
    metrics = dict(loss=o["loss"], policy_loss=o["policy_loss"], value_loss=o["value_loss"], entropy=o["entropy"],
                   approx_kl=float(np.mean(np.expm1(logratio) - logratio)), grad_norm=norm)
    return dict(params=dict(trunk=trunk.with_flat(new[:nt]), gru=tuple(new[nt:nt + 4]), head=tuple(new[nt + 4:])),
                S=S2, V=V2, metrics=metrics, grads=grads)


def recurrent_ppo_update(params: dict, rollout: dict, *, rng, minibatch_size: int, epochs: int, seq_len: int,
                         gamma: float = 0.99, lam: float = 0.95, batches_only: bool = False, **step_cfg) -> dict:
    """-> dict(params, steps, batches): the whole recurrent update
    (`batches_only`: the minibatches alone, no step taken)."""
    rewards = np.asarray(rollout["rewards"], np.float32)
    T, N = rewards.shape
    valid = rollout.get("valid")
    valid = np.ones((T, N), np.float32) if valid is None else np.asarray(valid, np.float32)
    adv, ret = gae(rewards, rollout["values"], rollout["dones"], rollout["last_values"], gamma, lam, valid)
    adv_n, _, _ = normalize_advantages(adv, valid)
    flat = dict(obs=np.asarray(rollout["obs"]).reshape((T * N,) + np.shape(rollout["obs"])[2:]),
                actions=np.asarray(rollout["actions"]).reshape(-1),
                old_logp=np.asarray(rollout["logp"], np.float64).reshape(-1),
                advantages=np.asarray(adv_n, np.float64).reshape(-1), returns=np.asarray(ret, np.float64).reshape(-1),
                values=np.asarray(rollout["values"], np.float64).reshape(-1), valid=valid.reshape(-1),
                starts=np.asarray(rollout["starts"], np.float64).reshape(-1))
    hidden = np.asarray(rollout["hidden"], np.float64).reshape(-1, np.shape(rollout["hidden"])[-1])
    flat_params = params["trunk"].flat() + list(params["gru"]) + list(params["head"])
    S = [np.zeros(np.shape(p)) for p in flat_params]
    V = [np.zeros(np.shape(p)) for p in flat_params]
    steps, batches = [], []
    for t, (rows, h0_rows) in enumerate(sequence_minibatches(T, N, seq_len, minibatch_size, epochs, rng), start=1):
        mb = {k: v[rows] for k, v in flat.items()}
        mb["h0"] = hidden[h0_rows]
        batches.append(mb)
        if batches_only:
            continue
        r = recurrent_ppo_step(params, S, V, t, mb, seq_len=seq_len, **step_cfg)
        params, S, V = r["params"], r["S"], r["V"]
        steps.append(r["metrics"])
    return dict(params=params, steps=steps, batches=batches)
