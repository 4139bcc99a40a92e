"""DQN and SAC as agents (the Agent protocol of ttrl/algos/base.py:118-187):
a learner, its GPU-resident replay, the update clock and the autoreset
bookkeeping, behind act / observe / should_update / update.

One gradient step (ttrl/algos/dqn/agent.py:183-214, ttrl/algos/sac/agent.py:218-238)
stays on the device end to end: the replay draws the batch and assembles it
straight into the learner's bound inputs, the captured update replays, one
copy brings the metrics back, and the prioritized write-back reads the TD
errors the update left on the device.  What crosses from the host is what
the reference draws on the host -- the sampler's generator draws and, for
SAC, the policy noise of the step (`rng.standard_normal`, in the
reference's order).

`update()` runs every step the clock owes (at least one), in order, and
returns the metrics averaged over them with `gradient_steps` (DQN also
`epsilon`).
"""

from __future__ import annotations

import numpy as np

from ttrl_amd.algos.base import AutoresetTracker, Transition, leaf_array
from ttrl_amd.algos.clock import UpdateClock
from ttrl_amd.algos.dqn import DQNConfig, DQNLearner, leaf_key
from ttrl_amd.algos.sac import SACConfig, SACLearner
from ttrl_amd.buffers.replay import ReplayBuffer, beta_at
from ttrl_amd.engine.ops import _kernels as K

__all__ = ["DQNAgent", "SACAgent"]


class _OffPolicyAgent:
    """What DQN and SAC share: the replay, the writer, the clock."""

    learner = None
    cfg = None

    def _setup(self, obs_spec, action_spec, device, n_envs: int, seed):
        cfg = self.cfg
        self.obs_spec, self.action_spec, self.device = obs_spec, action_spec, device
        self.n_envs = int(n_envs)
        self.priority = cfg.replay_priority()
        self.buffer = ReplayBuffer(obs_spec, action_spec, device, capacity=cfg.buffer_capacity, n_envs=self.n_envs,
                                   n_step=cfg.n_step, gamma=cfg.gamma, seed=seed, priority=self.priority,
                                   max_batch=max(1024, cfg.batch_size))
        self._clock = UpdateClock(cfg.train_freq, cfg.learning_starts)
        self._autoreset = AutoresetTracker(self.n_envs)

    # -- observing ---------------------------------------------------------

    def observe(self, transition: Transition) -> None:
        """Write the lanes of one vector-env step that are real transitions
        into replay, an ending lane's `next_obs` as its episode-final
        observation (ttrl/algos/offpolicy.py:37-58)."""
        real = np.flatnonzero(self._autoreset.valid(transition))
        if real.size == 0:
            return
        name = self.obs_spec.name
        obs = leaf_array(transition.obs, name)[real]
        nxt = leaf_array(transition.next_obs, name)[real]
        done = transition.done[real]
        self.buffer.add_lanes(real, obs, np.asarray(transition.action)[real], np.asarray(transition.reward)[real],
                              np.asarray(transition.terminated, bool)[real], np.asarray(transition.truncated, bool)[real],
                              final_obs=nxt if done.any() else None)

    def should_update(self, frame: int) -> bool:
        """The update clock at `frame` (ttrl/algos/dqn/agent.py:126-133):
        frames collected before a full batch is sampleable owe nothing."""
        if self.buffer.num_sampleable < self.cfg.batch_size:
            self._clock.skip(frame)
            return False
        self._clock.advance(frame)
        return self._clock.due

    def update(self) -> dict:
        steps = max(1, self._clock.owed)
        totals: dict = {}
        for _ in range(steps):
            for key, value in self._gradient_step().items():
                totals[key] = totals.get(key, 0.0) + value
        self._clock.consume(steps)
        out = {key: value / steps for key, value in totals.items()}
        out["gradient_steps"] = float(steps)
        return out

    def _beta(self):
        return None if self.priority is None else beta_at(self.priority, self.learner.update_count)

    # -- state ---------------------------------------------------------------

    def state_dict(self, *, weights_only: bool = False) -> dict:
        state = self.learner.state_dict(weights_only=weights_only)
        if not weights_only:
            state["autoreset"] = self._autoreset.state_dict()
            state["clock"] = self._clock.state_dict()
        return state

    def load_state_dict(self, state: dict, *, weights_only: bool = False) -> None:
        run = not (weights_only or state.get("weights_only", False))
        if run:
            missing = [k for k in ("autoreset", "clock") if k not in state]
            if missing:
                raise ValueError(f"{type(self).__name__}.load_state_dict: state is missing {missing}.")
        self.learner.load_state_dict(state, weights_only=weights_only)
        if run:
            self._autoreset.load_state_dict(state["autoreset"])
            self._clock.load_state_dict(state["clock"])

    def close(self) -> None:
        self.learner.close()


class DQNAgent(_OffPolicyAgent):
    """Double DQN with n-step returns and (optionally) prioritized replay
    (ttrl/algos/dqn/agent.py:38-253)."""

    def __init__(self, obs_spec, action_spec, device, *, cfg: DQNConfig = DQNConfig(), n_envs: int = 1,
                 seed: int | None = None):
        self.cfg = cfg
        self.learner = DQNLearner(obs_spec, action_spec, device, cfg=cfg, seed=seed, n_envs=n_envs)
        self._setup(obs_spec, action_spec, device, n_envs, seed)
        inp = self.learner.inputs
        leaf = obs_spec.name
        self._out = {"obs": inp[leaf_key("obs", leaf)].data, "next_obs": inp[leaf_key("next_obs", leaf)].data,
                     "actions_onehot": inp["actions_onehot"].data, "rewards": inp["rewards"].data,
                     "dones": inp["dones"].data, "discounts": inp["discounts"].data}
        if self.priority is not None:
            self._out["weights"] = inp["is_weights"].data

    @property
    def online(self):
        return self.learner.online

    @property
    def target(self):
        return self.learner.target

    def act(self, obs, *, deterministic: bool = False, episode_starts=None) -> np.ndarray:
        return self.learner.act(leaf_array(obs, self.obs_spec.name), deterministic=deterministic,
                                episode_starts=episode_starts)

    def epsilon(self) -> float:
        return self.learner.epsilon()

    def named_parameters(self):
        """The online network's parameters (the target is a lagged copy)."""
        return self.learner.online.named_parameters()

    def parameters(self):
        return self.learner.online.parameters()

    def update(self) -> dict:
        out = super().update()
        out["epsilon"] = self.learner.epsilon()
        return out

    def _gradient_step(self) -> dict:
        batch = self.buffer.sample(self.cfg.batch_size, beta=self._beta(), out=self._out)
        m = self.learner.update()
        if self.priority is not None:
            # |TD error| of the batch, read from the metric block on the device
            self.buffer.update_priorities_device(batch, self.learner._metrics_out["td_abs"])
        return {"loss": m["loss"], "mean_q": m["mean_q"], "grad_norm": m["grad_norm"]}


class SACAgent(_OffPolicyAgent):
    """SAC with twin critics, learned temperature, Polyak targets and an
    n-step replay (ttrl/algos/sac/agent.py:38-282)."""

    def __init__(self, obs_spec, action_spec, device, *, cfg: SACConfig = SACConfig(), n_envs: int = 1,
                 seed: int | None = None):
        self.cfg = cfg
        self.learner = SACLearner(obs_spec, action_spec, device, cfg=cfg, seed=seed, n_envs=n_envs)
        self._setup(obs_spec, action_spec, device, n_envs, seed)
        b = self.learner.batch
        self._out = {k: b[k].data for k in ("obs", "next_obs", "actions", "rewards", "dones", "discounts")}
        if self.priority is not None:
            self._out["weights"] = b["is_weights"].data
        self.obs_dim, self.act_dim = int(obs_spec.size), int(action_spec.dim)

    @property
    def nets(self):
        return self.learner.nets

    def act(self, obs, *, deterministic: bool = False, episode_starts=None) -> np.ndarray:
        return self.learner.act(leaf_array(obs, self.obs_spec.name), deterministic=deterministic,
                                episode_starts=episode_starts)

    def named_parameters(self):
        """The policy's and the critics' parameters and log_alpha (the
        targets are Polyak copies)."""
        yield from self.learner.nets.policy.named_parameters()
        for name, p in self.learner.nets.critics.named_parameters():
            yield f"critics.{name}", p
        yield "log_alpha", self.learner.log_alpha

    def parameters(self):
        for _, p in self.named_parameters():
            yield p

    def _gradient_step(self) -> dict:
        B, learner = self.cfg.batch_size, self.learner
        b = learner.batch
        batch = self.buffer.sample(B, beta=self._beta(), out=self._out)
        # the critic input concat(s, a), assembled next to the batch on the device
        K.copy_region(b["obs"].data, (0, 0), b["obs_actions"].data, (0, 0), (B, self.obs_dim))
        K.copy_region(b["actions"].data, (0, 0), b["obs_actions"].data, (0, self.obs_dim), (B, self.act_dim))
        # the policy noise of this step, from the agent's generator in the
        # reference's order (ttrl/algos/sac/agent.py:223-225)
        b.load("noise", learner._rng.standard_normal((B, self.act_dim)))
        b.load("next_noise", learner._rng.standard_normal((B, self.act_dim)))
        m = learner.update()
        if self.priority is not None:
            self.buffer.update_priorities_device(batch, learner._critic_out["td_abs"])
        keys = ("critic_loss", "actor_loss", "alpha_loss", "alpha", "entropy", "mean_q_target", "critic_grad_norm",
                "actor_grad_norm")
        return {k: float(m[k]) for k in keys}
