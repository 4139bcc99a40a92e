"""Seeded synthetic inputs and initial weights for the learner-update
workloads (uint8 Atari-shaped frames for DQN, Hopper-shaped vectors for SAC).

No data is downloaded: every array is drawn from numpy's default_rng with
the given seed, with the distributions of the benchmark configurations:
  DQN  frames uint8 uniform 0..255, actions uniform in [0, A), rewards in
       {-1, 0, 1} w.p. 0.05 / 0.9 / 0.05, done ~ Bernoulli(0.01), discounts
       gamma**n_step, importance weights uniform in (0.4, 1];
  SAC  observations and actions N(0, 1) (actions clipped to [-1, 1]),
       rewards N(0, 1), done ~ Bernoulli(0.001), reparameterisation noise
       N(0, 1).
Weights are He-uniform U(+-sqrt(6/fan_in)) with biases U(+-1/sqrt(fan_in)).
"""

from __future__ import annotations

import numpy as np

__all__ = ["dqn_batch", "sac_batch", "he_uniform_qnet_state", "he_uniform_sac_state"]


def dqn_batch(seed: int, batch: int = 32, num_actions: int = 6, frame_shape=(4, 84, 84), gamma: float = 0.99,
              n_step: int = 3, prioritized: bool = True, discounts=None) -> dict:
    rng = np.random.default_rng(seed)
    out = {
        "obs": rng.integers(0, 256, (batch,) + tuple(frame_shape), dtype=np.uint8),
        "next_obs": rng.integers(0, 256, (batch,) + tuple(frame_shape), dtype=np.uint8),
        "actions": rng.integers(0, num_actions, batch).astype(np.int64),
        "rewards": rng.choice(np.array([-1.0, 0.0, 1.0], np.float32), batch, p=[0.05, 0.9, 0.05]),
        "dones": (rng.random(batch) < 0.01).astype(np.float32),
        "discounts": (np.full(batch, gamma ** n_step, np.float32) if discounts is None
                      else np.asarray(discounts, np.float32)),
    }
    if prioritized:
        out["is_weights"] = (1.0 - 0.6 * rng.random(batch)).astype(np.float32)  # (0.4, 1]
    return out


def sac_batch(seed: int, batch: int = 256, obs_dim: int = 11, act_dim: int = 3, gamma: float = 0.99) -> dict:
    rng = np.random.default_rng(seed)
    return {
        "obs": rng.standard_normal((batch, obs_dim)).astype(np.float32),
        "next_obs": rng.standard_normal((batch, obs_dim)).astype(np.float32),
        "actions": np.clip(rng.standard_normal((batch, act_dim)), -1.0, 1.0).astype(np.float32),
        "rewards": rng.standard_normal(batch).astype(np.float32),
        "dones": (rng.random(batch) < 0.001).astype(np.float32),
        "discounts": np.full(batch, gamma, np.float32),
        "noise": rng.standard_normal((batch, act_dim)).astype(np.float32),
        "next_noise": rng.standard_normal((batch, act_dim)).astype(np.float32),
    }


def ppo_rollout(seed: int, n_steps: int = 128, n_envs: int = 8, num_actions: int = 18,
                frame_shape=(4, 84, 84)) -> dict:
    """One synthetic PPO rollout, time-major [T, N]: uint8 frames uniform
    0..255, actions uniform, rewards in {-1, 0, 1} w.p. 0.05/0.9/0.05,
    dones Bernoulli(0.01), values and last values N(0, 1), and the behaviour
    policy's log-probs of the actions under random logits."""
    rng = np.random.default_rng(seed)
    T, N = n_steps, n_envs
    logits = rng.standard_normal((T, N, num_actions))
    actions = rng.integers(0, num_actions, (T, N))
    lse = np.log(np.exp(logits - logits.max(-1, keepdims=True)).sum(-1)) + logits.max(-1)
    logp = np.take_along_axis(logits, actions[..., None], -1)[..., 0] - lse
    return {
        "obs": rng.integers(0, 256, (T, N) + tuple(frame_shape), dtype=np.uint8),
        "actions": actions,
        "rewards": rng.choice(np.array([-1.0, 0.0, 1.0], np.float32), (T, N), p=[0.05, 0.9, 0.05]),
        "dones": (rng.random((T, N)) < 0.01).astype(np.float32),
        "values": rng.standard_normal((T, N)).astype(np.float32),
        "logp": logp.astype(np.float32),
        "last_values": rng.standard_normal(N).astype(np.float32),
    }


def recurrent_ppo_rollout(seed: int, n_steps: int = 128, n_envs: int = 16, num_actions: int = 18,
                          seq_len: int = 32, hidden_size: int = 512, frame_shape=(4, 84, 84)) -> dict:
    """ppo_rollout plus what a recurrent update reads: `starts` [T, N] (the
    previous step's done shifted by one, the first row from Bernoulli(0.01)
    carried flags) and `hidden` [T / seq_len, N, hidden] states entering each
    sequence, N(0, 0.5)."""
    out = ppo_rollout(seed, n_steps, n_envs, num_actions, frame_shape)
    rng = np.random.default_rng(seed + 1)
    starts = np.zeros((n_steps, n_envs), np.float32)
    starts[0] = (rng.random(n_envs) < 0.01).astype(np.float32)
    starts[1:] = out["dones"][:-1]
    out["starts"] = starts
    out["hidden"] = (0.5 * rng.standard_normal((n_steps // seq_len, n_envs, hidden_size))).astype(np.float32)
    return out


def _he(rng, shape, fan_in):
    bound = np.sqrt(6.0 / fan_in)
    return rng.uniform(-bound, bound, shape).astype(np.float32)


def _bias(rng, n, fan_in):
    bound = 1.0 / np.sqrt(fan_in)
    return rng.uniform(-bound, bound, n).astype(np.float32)


def he_uniform_qnet_state(net, seed: int) -> dict:
    """A state_dict for `net` (a built Q network) with He-uniform weights."""
    rng = np.random.default_rng(seed)
    state = {}
    ref = net.state_dict()
    keys = list(ref)
    for k in keys:
        shape = ref[k].shape
        if k.endswith("weight"):
            fan_in = int(np.prod(shape[1:])) if len(shape) == 4 else int(shape[0])
            state[k] = _he(rng, shape, fan_in)
            last_fan = fan_in
        else:
            state[k] = _bias(rng, int(np.prod(shape)), last_fan).reshape(shape)
    return state


def he_uniform_sac_state(module, seed: int) -> dict:
    """He-uniform weights for any module of Linear layers (W stored (in, out))."""
    rng = np.random.default_rng(seed)
    state = {}
    ref = module.state_dict()
    last_fan = 1
    for k, v in ref.items():
        if k.endswith("weight"):
            last_fan = int(v.shape[0])
            state[k] = _he(rng, v.shape, last_fan)
        else:
            state[k] = _bias(rng, int(np.prod(v.shape)), last_fan).reshape(v.shape)
    return state
