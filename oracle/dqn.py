"""Float64 restatement of one DQN learner update.

update_loss   ttrl/algos/dqn/losses.py:77-140 (double-DQN selection with the
              online net, valuation with the target net, n-step target
              r + discounts*(1 - done)*Q', Huber through the clipped-quadratic
              identity ttrl/engine/ops/functional.py:56-69, importance weights
              before the mean, metrics loss / mean_q / td_abs / grad_sq)
argmax        first index of the maximum (ttrl/engine/ops/reduce.py:82-99)
Adam step     oracle.adam.fused_step (ttrl/engine/optim/adam.py:93-134), t = 1
grad_norm     sqrt(sum g^2) over the online parameters (ttrl/algos/dqn/agent.py:209-213)
"""

from __future__ import annotations

import numpy as np

from oracle import adam, fa, float_type
from oracle.nets import GateStats, QNet, qnet_backward, qnet_forward

ARGMAX_BAND = 1e-4


def select_actions(q_sel: np.ndarray, device_actions=None, band: float = ARGMAX_BAND):
    """argmax per row; where the top-two gap is within `band` of the row's
    scale the device's choice is adopted (ttrl: tests/hardware/test_deploy_parity.py:281-292)."""
    a = np.argmax(q_sel, axis=1)
    adopted = 0
    if device_actions is not None:
        dev = np.asarray(device_actions).reshape(-1).astype(np.int64)
        srt = np.sort(q_sel, axis=1)
        gap = srt[:, -1] - srt[:, -2] if q_sel.shape[1] > 1 else np.full(q_sel.shape[0], np.inf)
        scale = np.maximum(np.abs(srt[:, -1]), 1e-30)
        close = gap <= band * scale
        chosen_ok = q_sel[np.arange(len(dev)), dev] >= srt[:, -1] - band * scale
        take = close & chosen_ok & (dev != a)
        adopted = int(np.sum(take))
        a = np.where(take, dev, a)
    return a, adopted


def huber(e: np.ndarray, delta: float) -> np.ndarray:
    ae = np.abs(e)
    quad = np.minimum(ae, delta)
    return 0.5 * quad * quad + delta * (ae - quad)


def dqn_update(online: QNet, target: QNet, batch: dict, *, double: bool = True, delta: float = 1.0,
               lr: float = 6.25e-5, eps: float = 1.5e-4, betas=(0.9, 0.999), gates=None,
               device_next_actions=None, prioritized: bool = True, adam_state=None, t: int = 1) -> dict:
    """One update; every array float64.  The Adam step starts from
    `adam_state` = (S list, V list) in the online parameters' order at update
    count `t` (1-based), or from zero moments at t = 1."""
    stats = GateStats()
    obs, nxt = batch["obs"], batch["next_obs"]
    actions = np.asarray(batch["actions"]).reshape(-1).astype(np.int64)
    B = obs.shape[0]
    q, acts = qnet_forward(online, obs, gates=gates, stats=stats)
    A = q.shape[1]
    q_online_next, _ = qnet_forward(online, nxt)
    q_target_next, _ = qnet_forward(target, nxt)
    sel = q_online_next if double else q_target_next
    a_star, adopted = select_actions(sel, device_next_actions)
    nv = q_target_next[np.arange(B), a_star]
    rewards = fa(batch["rewards"]).reshape(-1)
    dones = fa(batch["dones"]).reshape(-1)
    discounts = fa(batch["discounts"]).reshape(-1)
    y = rewards + discounts * (1.0 - dones) * nv
    pred = q[np.arange(B), actions]
    e = pred - y
    w = fa(batch["is_weights"]).reshape(-1) if prioritized else np.ones(B, float_type())
    loss = float(np.mean(w * huber(e, delta)))
    dq = np.zeros((B, A), float_type())
    dq[np.arange(B), actions] = w / B * np.clip(e, -delta, delta)
    grads = qnet_backward(online, acts, dq)
    grad_sq = float(sum(np.sum(g * g) for g in grads))
    b1, b2 = betas
    new, new_S, new_V = [], [], []
    for i, (p, g) in enumerate(zip(online.flat(), grads)):
        S0 = np.zeros_like(g) if adam_state is None else fa(adam_state[0][i]).reshape(g.shape)
        V0 = np.zeros_like(g) if adam_state is None else fa(adam_state[1][i]).reshape(g.shape)
        p1, S1, V1 = adam.fused_step(p, g, S0, V0, t, lr, b1, b2, eps)
        new.append(p1)
        new_S.append(S1)
        new_V.append(V1)
    return {
        "q": q, "pred": pred, "q_online_next": q_online_next, "q_target_next": q_target_next,
        "next_actions": a_star, "td_target": y, "loss": loss, "mean_q": float(np.mean(pred)),
        "td_abs": np.abs(e), "dq": dq, "grads": grads, "grad_sq": grad_sq,
        "grad_norm": float(np.sqrt(grad_sq)), "new_params": new, "new_S": new_S, "new_V": new_V, "gate_stats": stats,
        "argmax_adopted": adopted,
    }
