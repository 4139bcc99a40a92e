"""DQN, SAC and PPO as agents (the Agent protocol of ttrl/algos/base.py:118-187):
a learner, its experience storage (GPU-resident replay; PPO's rollout), the
update clock and the autoreset bookkeeping, behind act / observe /
should_update / update.  Each constructor takes the keywords the
reference's `build_agent` passes (cfg, n_envs, seed, profile) and the
engine config.

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
from ttrl_amd.algos.ppo import PPOConfig, PPOLearner
from ttrl_amd.algos.sac import SACConfig, SACLearner
from ttrl_amd.buffers.replay import ReplayBuffer, beta_at
from ttrl_amd.engine.config import DEFAULT, EngineConfig, check_engine_config
from ttrl_amd.engine.ops import _kernels as K

__all__ = ["DQNAgent", "PPOAgent", "SACAgent"]


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
                 seed: int | None = None, profile=None, engine: EngineConfig = DEFAULT):
        self.cfg = cfg
        self.profile = profile
        self.engine = check_engine_config(engine, "DQNAgent")
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
                 seed: int | None = None, profile=None, engine: EngineConfig = DEFAULT):
        self.cfg = cfg
        self.profile = profile
        self.engine = check_engine_config(engine, "SACAgent")
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


class PPOAgent:
    """Clipped PPO over a shared-trunk actor-critic with a categorical
    policy (ttrl/algos/ppo/agent.py:40-238, ttrl/algos/ppo/learn.py:46-112).

    `act` runs the captured acting forward at the lane count (log-softmax
    of the logits and the value on the device) and draws each lane's action
    on the host by the reference's inverse-CDF rule against one uniform per
    lane (ttrl/algos/ppo/policy.py:37-62), recording the log-prob and value
    for `observe`.  `observe` appends one vector step to the host rollout
    (autoreset padding steps stored with valid 0); `should_update` is true
    once the rollout holds n_steps steps; `update` bootstraps V of the last
    next observation, then the learner uploads the rollout, runs GAE and
    every epoch's minibatch steps on the device, and the rollout resets.
    Feedforward policies only: a recurrent config is refused."""

    def __init__(self, obs_spec, action_spec, device, *, cfg: PPOConfig = PPOConfig(), n_envs: int = 1,
                 seed: int | None = None, profile=None, engine: EngineConfig = DEFAULT, boundaries=None):
        from ttrl_amd.nets.acting import ActingNet, CategoricalValueDecision

        if cfg.recurrent is not None:
            raise ValueError("PPOAgent: a recurrent PPOConfig is not supported by the agent; drive "
                             "RecurrentPPOLearner.update(rollout) with sequences of your own instead")
        if boundaries is not None:
            raise ValueError("PPOAgent: episode boundaries only matter to a recurrent policy, and this agent "
                             "builds feedforward ones; pass boundaries=None")
        if int(n_envs) < 1:
            raise ValueError(f"PPOAgent: n_envs must be >= 1, got {n_envs}")
        if cfg.minibatch_size > cfg.n_steps * int(n_envs):
            raise ValueError(f"PPO: minibatch_size={cfg.minibatch_size} exceeds the {cfg.n_steps * int(n_envs)} "
                             f"transitions one rollout collects (n_steps={cfg.n_steps} x n_envs={n_envs}), so no "
                             f"minibatch could ever be drawn")
        if int(n_envs) > cfg.minibatch_size:
            raise ValueError(f"PPO: n_envs={n_envs} exceeds the network batch minibatch_size="
                             f"{cfg.minibatch_size}; acting runs the network at the lane count")
        self.cfg = cfg
        self.profile = profile
        self.engine = check_engine_config(engine, "PPOAgent")
        self.obs_spec, self.action_spec, self.device = obs_spec, action_spec, device
        self.n_envs = int(n_envs)
        self.num_actions = int(action_spec.n)
        self.learner = PPOLearner(obs_spec, action_spec, device, cfg=cfg, seed=seed)
        self._acting = ActingNet(self.learner.net, obs_spec, device, width=cfg.minibatch_size, lanes=self.n_envs,
                                 decision=CategoricalValueDecision(), mode="graph")
        self._autoreset = AutoresetTracker(self.n_envs)
        self._rng = np.random.default_rng(seed)
        self._eval_rng = np.random.default_rng(seed).spawn(1)[0]
        self._pending = None
        self._last_next_obs = None
        T, N = cfg.n_steps, self.n_envs
        leaf = tuple(obs_spec.shape) if obs_spec.kind == "image" else (obs_spec.size,)
        frames = np.uint8 if obs_spec.kind == "image" else np.float32
        self._rollout = {"obs": np.zeros((T, N) + leaf, frames), "actions": np.zeros((T, N), np.int64),
                         "logp": np.zeros((T, N), np.float32), "values": np.zeros((T, N), np.float32),
                         "rewards": np.zeros((T, N), np.float32), "dones": np.zeros((T, N), np.float32),
                         "valid": np.zeros((T, N), np.float32)}
        self._t = 0

    @property
    def net(self):
        return self.learner.net

    @property
    def optimizer(self):
        return self.learner.optimizer

    @property
    def frame_count(self) -> int:
        return self.learner.frame_count

    @property
    def update_count(self) -> int:
        return self.learner.update_count

    # -- acting --------------------------------------------------------------

    def act(self, obs, *, deterministic: bool = False, episode_starts=None) -> np.ndarray:
        """One action per lane; a stochastic step records its log-prob and
        value for the `observe` that follows.  `episode_starts` belongs to
        the acting contract of a policy with memory; this one has none."""
        out = self._acting.decide(leaf_array(obs, self.obs_spec.name))
        logp_all = out["logp"]
        batch = logp_all.shape[0]
        if deterministic:
            actions = np.argmax(logp_all, axis=-1)
        else:
            probs = np.exp(logp_all)
            probs = probs / probs.sum(axis=-1, keepdims=True)
            cdf = np.cumsum(probs, axis=-1)
            actions = (self._rng.random(batch)[:, None] > cdf).sum(axis=-1)
            actions = np.clip(actions, 0, self.num_actions - 1)
        actions = actions.astype(np.int64)
        if not deterministic:
            self._pending = {"action": actions, "logp": logp_all[np.arange(batch), actions].astype(np.float32),
                             "value": out["value"].reshape(-1)[:batch].astype(np.float32)}
        return actions

    # -- observing -----------------------------------------------------------

    def observe(self, transition: Transition) -> None:
        """Append one vector step, padding steps included with valid 0
        (ttrl/algos/ppo/agent.py:138-189)."""
        if self._pending is None:
            raise RuntimeError("PPO.observe: no act() preceded this transition. PPO records the log-prob and the "
                               "value from the forward pass that chose the action, so every observe must follow "
                               "the act that produced it; a deterministic act (evaluation) records nothing and "
                               "must not be fed back.")
        valid = self._autoreset.valid(transition)
        pending, self._pending = self._pending, None
        if pending["logp"].shape[0] != transition.n_envs:
            raise ValueError(f"PPO.observe: the last act() produced {pending['logp'].shape[0]} actions but this "
                             f"transition has {transition.n_envs} lanes")
        if self._t >= self.cfg.n_steps:
            raise RuntimeError(f"PPO.observe: the rollout already holds its {self.cfg.n_steps} steps; call "
                               f"update() when should_update() says so")
        t, r = self._t, self._rollout
        r["obs"][t] = leaf_array(transition.obs, self.obs_spec.name)
        r["actions"][t] = pending["action"]
        r["logp"][t] = pending["logp"]
        r["values"][t] = pending["value"]
        r["rewards"][t] = np.asarray(transition.reward, np.float32)
        r["dones"][t] = np.asarray(transition.terminated, np.float32)
        r["valid"][t] = valid.astype(np.float32)
        self._t += 1
        self._last_next_obs = leaf_array(transition.next_obs, self.obs_spec.name)
        self.learner.frame_count += transition.n_envs

    def should_update(self, frame: int) -> bool:
        """A full rollout: the trigger is how much this policy collected."""
        return self._t >= self.cfg.n_steps

    # -- learning ------------------------------------------------------------

    def _last_values(self) -> np.ndarray:
        """V(s) of the observation after the rollout's last stored step."""
        out = self._acting.decide(self._last_next_obs)
        return out["value"].reshape(-1)[:self.n_envs].astype(np.float32)

    def update(self) -> dict:
        if self._t < self.cfg.n_steps:
            raise RuntimeError(f"PPO.update: the rollout holds fewer than its {self.cfg.n_steps} steps. Gate on "
                               f"should_update, which reports when it is full.")
        rollout = dict(self._rollout)
        rollout["last_values"] = self._last_values()
        metrics = self.learner.update(rollout)
        self._t = 0
        return metrics

    def named_parameters(self):
        """The whole actor-critic: on-policy learning keeps no lagged copy."""
        return self.learner.net.named_parameters()

    def parameters(self):
        return self.learner.net.parameters()

    # -- state -----------------------------------------------------------------

    def _rollout_state(self) -> dict:
        t = self._t
        state = {"t": t, "acting_rng": self._rng.bit_generator.state,
                 "last_next_obs": None if self._last_next_obs is None else np.array(self._last_next_obs)}
        state.update({k: v[:t].copy() for k, v in self._rollout.items()})
        return state

    def state_dict(self, *, weights_only: bool = False) -> dict:
        """The learner's tree (net, config, optimizer, counters, the
        shuffle generator) plus the run state the agent holds: autoreset
        phase and the half-collected rollout with the acting generator."""
        state = self.learner.state_dict(weights_only=weights_only)
        if not weights_only:
            state["autoreset"] = self._autoreset.state_dict()
            state["rollout"] = self._rollout_state()
        return state

    def load_state_dict(self, state: dict, *, weights_only: bool = False) -> None:
        run = not (weights_only or state.get("weights_only", False))
        if run:
            missing = [k for k in ("autoreset", "rollout") if k not in state]
            if missing:
                raise ValueError(f"PPOAgent.load_state_dict: state is missing {missing}.")
        self.learner.load_state_dict(state, weights_only=weights_only)
        self._pending = None
        if not run:
            self._t = 0
            return
        self._autoreset.load_state_dict(state["autoreset"])
        ro = state["rollout"]
        t = int(ro["t"])
        if not 0 <= t <= self.cfg.n_steps:
            raise ValueError(f"PPOAgent.load_state_dict: the stored rollout holds {t} steps; this agent's "
                             f"n_steps is {self.cfg.n_steps}")
        for k, v in self._rollout.items():
            arr = np.asarray(ro[k])
            if arr.shape != (t,) + v.shape[1:]:
                raise ValueError(f"PPOAgent.load_state_dict: stored rollout field {k!r} has shape {arr.shape}, "
                                 f"expected {(t,) + v.shape[1:]}")
            v[:t] = arr
        self._t = t
        self._rng.bit_generator.state = ro["acting_rng"]
        last = ro.get("last_next_obs")
        self._last_next_obs = None if last is None else np.asarray(last)

    def close(self) -> None:
        self._acting.close()
        self.learner.close()
