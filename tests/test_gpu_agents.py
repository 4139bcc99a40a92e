"""DQN and SAC agents through the Agent protocol (ttrl/algos/base.py:118-187)
on the GPU: rounds of act -> observe -> should_update -> update() over a
synthetic vector env with episode ends and NEXT_STEP autoreset padding.

Each agent runs in lockstep with a twin learner fed the replay oracle's
batches (oracle/replay.py, driven with the same real transitions and seed):
the agent's device-side draw, assembly into the bound inputs, policy noise
and prioritized write-back must reproduce the twin's update bit for bit
(metrics, every parameter, the target / Polyak copies, log_alpha) and the
oracle's priority table (rel 1e-12).  The DQN twin is in turn checked at
every step against the float64 oracle (oracle/dqn.py) from its own
parameters and Adam moments, with the device's ReLU gates and argmax
choices adopted inside the stated bands: loss, mean_q, grad_norm and the
updated parameters at rel 1e-4.
"""

from __future__ import annotations

from dataclasses import replace

import numpy as np
import pytest

from tests._dqn_helpers import adam_moments as _adam_moments

pytestmark = pytest.mark.gpu

SHAPE = (4, 36, 36)  # the Nature CNN's strides take 36 -> 8 -> 3 -> 1


def _env_step(rng, L, pending, p_term=0.06, p_trunc=0.03):
    """Flags of one vector step: a lane on its autoreset step reports no end."""
    x = rng.random(L)
    term = (x < p_term) & ~pending
    trunc = (~term) & (x < p_term + p_trunc) & ~pending
    return term, trunc


def test_dqn_agent_rounds_match_twin_and_oracle(device):
    from oracle.dqn import dqn_update
    from oracle.nets import qnet_forward
    from oracle.replay import ReplayOracle
    from tests._dqn_helpers import qnet_to_oracle
    from ttrl_amd.algos.agents import DQNAgent
    from ttrl_amd.algos.base import Agent, Transition
    from ttrl_amd.algos.dqn import DQNConfig, DQNLearner
    from ttrl_amd.buffers import PriorityConfig, beta_at
    from ttrl_amd.engine import layers
    from ttrl_amd.spaces import ActionSpec, ObsSpec
    from ttrl_amd.workloads import he_uniform_qnet_state

    L, B, A, seed = 2, 16, 6, 5
    prio = PriorityConfig(alpha=0.6, beta_anneal_updates=40)
    cfg = DQNConfig(lr=6.25e-5, adam_eps=1.5e-4, batch_size=B, prioritized=True, priority=prio, n_step=3,
                    buffer_capacity=160, train_freq=2, learning_starts=30, target_sync_interval=3)
    spec, aspec = ObsSpec.image(SHAPE), ActionSpec.discrete(A)
    agent = DQNAgent(spec, aspec, device, cfg=cfg, n_envs=L, seed=seed)
    twin = DQNLearner(spec, aspec, device, cfg=replace(cfg, step_mode="eager"), seed=seed, n_envs=L)
    assert isinstance(agent, Agent)
    try:
        online = he_uniform_qnet_state(agent.online, 9)
        rng0 = np.random.default_rng(10)
        target = {k: (v + 0.05 * np.abs(v).max() * rng0.standard_normal(v.shape)).astype(np.float32)
                  for k, v in online.items()}
        for net in (agent, twin):
            net.online.load_state_dict(online)
            net.target.load_state_dict(target)
        orc = ReplayOracle(SHAPE, np.uint8, capacity=160, n_envs=L, n_step=3, gamma=0.99, seed=seed, alpha=0.6,
                           epsilon=prio.epsilon)
        rng = np.random.default_rng(0)
        obs = rng.integers(0, 256, (L,) + SHAPE, dtype=np.uint8)
        pending = np.zeros(L, bool)
        frame, updates = 0, 0
        names = [n for n, _ in agent.named_parameters()]
        assert names == list(agent.online.state_dict().keys())
        for _ in range(64):
            actions = agent.act(obs)
            rewards = rng.choice([-1.0, 0.0, 1.0], L, p=[0.1, 0.8, 0.1]).astype(np.float32)
            term, trunc = _env_step(rng, L, pending)
            nxt = rng.integers(0, 256, (L,) + SHAPE, dtype=np.uint8)
            agent.observe(Transition(obs, actions, rewards, term, trunc, nxt))
            for lane in np.flatnonzero(~pending):
                ended = bool(term[lane] or trunc[lane])
                orc.add(lane, obs[lane], actions[lane], rewards[lane], term[lane], trunc[lane],
                        nxt[lane] if ended else None)
            pending = term | trunc
            reset = rng.integers(0, 256, (L,) + SHAPE, dtype=np.uint8)
            obs = np.where(pending[:, None, None, None], reset, nxt)
            frame += L
            if not agent.should_update(frame):
                continue
            # the twin's state before the step, for the float64 oracle
            p0 = twin.online.state_dict()
            t0 = twin.target.state_dict()
            S0, V0 = _adam_moments(twin.optimizer, twin.online)
            t_step = twin.optimizer.t + 1  # the update count this step runs at
            m = agent.update()
            assert m["gradient_steps"] == 1.0
            assert m["epsilon"] == agent.epsilon()
            ob = orc.sample(B, beta=beta_at(prio, updates))
            batch = {k: ob[k] for k in ("obs", "next_obs", "actions", "rewards", "dones", "discounts")}
            batch["is_weights"] = ob["weights"]
            layers.RECORD = []
            try:
                tm = twin.update(batch)
                recs = [[y.numpy() for y in ys] for ys in layers.RECORD[-5:]]
            finally:
                layers.RECORD = None
            # agent == twin, bit for bit
            for key in ("loss", "mean_q", "grad_norm"):
                assert m[key] == tm[key], (updates, key)
            for got, want in ((agent.online, twin.online), (agent.target, twin.target)):
                for k, v in want.state_dict().items():
                    assert np.array_equal(got.state_dict()[k], v), (updates, k)
            orc.update_priorities(ob["lanes"], ob["cols"], tm["td_abs"])
            table = agent.buffer.priorities_numpy()
            assert np.max(np.abs(table - orc.weight)) <= 1e-12 * orc.weight.max()
            # the twin's step against the float64 oracle
            onet, tnet = qnet_to_oracle(p0), qnet_to_oracle(t0)
            _, acts = qnet_forward(onet, batch["obs"])
            gates = {n: (recs[i][0] > 0).reshape(acts[i][1].shape)
                     for i, n in enumerate(("conv0", "conv1", "conv2", "fc0"))}
            ref = dqn_update(onet, tnet, batch, lr=cfg.lr, eps=cfg.adam_eps, gates=gates,
                             device_next_actions=np.argmax(recs[4][1], 1), adam_state=(S0, V0), t=t_step)
            for key in ("loss", "mean_q", "grad_norm"):
                assert abs(tm[key] - ref[key]) <= 1e-4 * max(abs(ref[key]), 1e-6), (updates, key)
            for (k, v), want in zip(twin.online.state_dict().items(), ref["new_params"]):
                err = np.max(np.abs(np.asarray(v, np.float64).reshape(want.shape) - want)) / np.max(np.abs(want))
                assert err < 1e-4, (updates, k, err)
            updates += 1
        assert updates >= 10
        # target syncs every 3 updates: after the last sync the target equals that step's online net
        assert agent.learner.update_count == updates
    finally:
        agent.close()
        twin.close()


def test_sac_agent_rounds_match_twin(device):
    from oracle.replay import ReplayOracle
    from ttrl_amd.algos.agents import SACAgent
    from ttrl_amd.algos.base import Agent, Transition
    from ttrl_amd.algos.sac import SACConfig, SACLearner
    from ttrl_amd.spaces import ActionSpec, ObsSpec
    from ttrl_amd.workloads import he_uniform_sac_state

    L, B, d, seed = 2, 32, 3, 7
    cfg = SACConfig(batch_size=B, buffer_capacity=200, train_freq=2, learning_starts=40)
    spec, aspec = ObsSpec.vector(11), ActionSpec.continuous(d)
    agent = SACAgent(spec, aspec, device, cfg=cfg, n_envs=L, seed=seed)
    twin = SACLearner(spec, aspec, device, cfg=cfg, seed=seed, n_envs=L)
    assert isinstance(agent, Agent)
    try:
        pol = he_uniform_sac_state(agent.nets.policy, 11)
        crit = he_uniform_sac_state(agent.nets.critics, 12)
        for net in (agent.nets, twin.nets):
            net.policy.load_state_dict(pol)
            net.critics.load_state_dict(crit)
            net.targets.load_state_dict(crit)
        orc = ReplayOracle((11,), np.float32, capacity=200, n_envs=L, n_step=1, gamma=0.99, seed=seed,
                           action_dim=d)
        mirror = np.random.default_rng(seed)  # the agent's generator: acting noise, then each step's noise
        rng = np.random.default_rng(1)
        obs = rng.standard_normal((L, 11)).astype(np.float32)
        pending = np.zeros(L, bool)
        frame, updates = 0, 0
        for _ in range(60):
            actions = agent.act(obs)
            mirror.standard_normal((L, d))
            rewards = rng.standard_normal(L).astype(np.float32)
            term, trunc = _env_step(rng, L, pending, 0.04, 0.02)
            nxt = rng.standard_normal((L, 11)).astype(np.float32)
            agent.observe(Transition(obs, actions, rewards, term, trunc, nxt))
            for lane in np.flatnonzero(~pending):
                ended = bool(term[lane] or trunc[lane])
                orc.add(lane, obs[lane], actions[lane], rewards[lane], term[lane], trunc[lane],
                        nxt[lane] if ended else None)
            pending = term | trunc
            obs = np.where(pending[:, None], rng.standard_normal((L, 11)).astype(np.float32), nxt)
            frame += L
            if not agent.should_update(frame):
                continue
            m = agent.update()
            assert m["gradient_steps"] == 1.0
            ob = orc.sample(B)
            batch = {k: ob[k] for k in ("obs", "next_obs", "actions", "rewards", "dones", "discounts")}
            batch["noise"] = mirror.standard_normal((B, d))
            batch["next_noise"] = mirror.standard_normal((B, d))
            tm = twin.update(batch)
            for key in ("critic_loss", "actor_loss", "alpha_loss", "alpha", "entropy", "mean_q_target",
                        "critic_grad_norm", "actor_grad_norm"):
                assert m[key] == tm[key], (updates, key)
            want = twin.nets.state_dict()
            got = agent.nets.state_dict()
            for k in want:
                assert np.array_equal(got[k], want[k]), (updates, k)
            assert np.array_equal(agent.learner.log_alpha.numpy(), twin.log_alpha.numpy())
            updates += 1
        assert updates >= 8
        names = [n for n, _ in agent.named_parameters()]
        assert names[-1] == "log_alpha" and len(names) == len(list(agent.parameters()))
    finally:
        agent.close()
        twin.close()


def test_agent_state_round_trip_keeps_clock_and_autoreset(device):
    from ttrl_amd.algos.agents import DQNAgent
    from ttrl_amd.algos.base import Transition
    from ttrl_amd.algos.dqn import DQNConfig
    from ttrl_amd.spaces import ActionSpec, ObsSpec

    cfg = DQNConfig(batch_size=8, buffer_capacity=64, train_freq=3, learning_starts=4)
    spec = ObsSpec.image(SHAPE)
    a = DQNAgent(spec, ActionSpec.discrete(4), device, cfg=cfg, n_envs=2, seed=1)
    b = DQNAgent(spec, ActionSpec.discrete(4), device, cfg=cfg, n_envs=2, seed=2)
    try:
        rng = np.random.default_rng(3)
        obs = rng.integers(0, 256, (2,) + SHAPE, dtype=np.uint8)
        for f in range(1, 12):
            nxt = rng.integers(0, 256, (2,) + SHAPE, dtype=np.uint8)
            a.observe(Transition(obs, np.array([1, 2]), np.zeros(2, np.float32), np.array([False, f == 5]),
                                 np.zeros(2, bool), nxt))
            a.should_update(2 * f)
            obs = nxt
        state = a.state_dict()
        assert state["clock"] == a._clock.state_dict() and "autoreset" in state
        b.load_state_dict(state)
        assert b._clock.state_dict() == a._clock.state_dict()
        assert not b._autoreset.pending.any()  # a restored run starts with no lane pending
        w = a.state_dict(weights_only=True)
        assert "clock" not in w
        b.load_state_dict(w, weights_only=True)
        broken = dict(state)
        del broken["clock"]
        with pytest.raises(ValueError, match="missing"):
            b.load_state_dict(broken)
    finally:
        a.close()
        b.close()
