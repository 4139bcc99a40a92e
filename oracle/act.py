"""Float64 restatement of the acting step either side of an update.

Test infrastructure only: the product's acting path never imports this.

epsilon        linear schedule eps_start -> eps_end over eps_decay_frames
               (ttrl/algos/dqn/agent.py:92-95)
dqn_act        greedy action = first-index argmax of the online Q row
               (ttrl/engine/ops/reduce.py:82-99); epsilon-greedy with the host
               draws in the reference's order: rng.random(batch), then
               rng.integers(0, A, size=batch), then where(draw < eps, random,
               greedy) (ttrl/algos/dqn/agent.py:97-119)
sac_act        policy forward (oracle.sac.policy_forward), then the squashed
               sample at rng.standard_normal((batch, d)), or tanh(mean) with
               logp 0 when deterministic, mapped onto the action bounds
               (ttrl/algos/sac/agent.py:111-125, ttrl/algos/sac/policy.py:42-59)
"""

from __future__ import annotations

import numpy as np

from oracle import gaussian
from oracle.dqn import select_actions
from oracle.nets import QNet, qnet_forward
from oracle.sac import SacParams, policy_forward


def epsilon(frame_count: int, eps_start: float, eps_end: float, eps_decay_frames: int) -> float:
    frac = min(1.0, frame_count / eps_decay_frames)
    return eps_start + frac * (eps_end - eps_start)


def epsilon_greedy(greedy, num_actions: int, eps: float, rng) -> np.ndarray:
    greedy = np.asarray(greedy).reshape(-1)
    batch = greedy.shape[0]
    draws = rng.random(batch)
    random_actions = rng.integers(0, num_actions, size=batch)
    return np.where(draws < eps, random_actions, greedy).astype(np.int64)


def dqn_act(net: QNet, frames, *, eps: float, rng, device_greedy=None):
    """-> (actions int64 (B,), q float64 (B, A), greedy int64 (B,), adopted)."""
    q, _ = qnet_forward(net, np.asarray(frames))
    greedy, adopted = select_actions(q, device_greedy)
    return epsilon_greedy(greedy, q.shape[1], eps, rng), q, greedy, adopted


def sac_act(P: SacParams, obs, *, rng=None, deterministic: bool = False, centre=0.0, half_width=1.0,
            log_det: float = 0.0):
    """-> (action (B, d), logp (B,), mean, clamped log_std); float64."""
    mean, _raw, log_std, _h, _acts = policy_forward(P, np.asarray(obs, np.float64))
    if deterministic:
        action = centre + half_width * np.tanh(mean)
        return action, np.zeros(mean.shape[0]), mean, log_std
    noise = rng.standard_normal(mean.shape)
    action, logp, _u = gaussian.sample(mean, log_std, noise, centre, half_width, log_det)
    return action, logp, mean, log_std
