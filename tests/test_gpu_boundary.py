"""The reference's entry sequence on the GPU: `with acquire(0) as (device,
profile)` (ttrl/engine/device/acquire.py:55-75, as ttrl/train/run.py:68 calls
it), then `resolve_and_build(name, obs_spec, action_spec, device, **kwargs)`
(ttrl/algos/registry.py:39-51, with the keywords ttrl/train/builders.py:139-144
passes), then rounds of act / observe / should_update / update.

DQN: the registry-built agent equals an agent constructed directly with the
same seed and fed the same transitions, bit for bit (metrics and every
parameter); the DQN agent itself is pinned against the float64 oracle step by
step in test_gpu_agents.py.

PPO: the acting outputs (log-softmax of the logits and the value per lane)
match the float64 oracle's forward at rel 1e-4; each stochastic action is the
reference's inverse-CDF draw against one uniform per lane from the agent's
generator (ttrl/algos/ppo/policy.py:37-62), replayed on the host; the update
equals PPOLearner.update on the rollout the agent collected, bit for bit
(metrics and every parameter), which test_gpu_ppo_update.py pins against the
float64 oracle.
"""

from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

SHAPE = (4, 36, 36)  # the Nature CNN's strides take 36 -> 8 -> 3 -> 1


def _env_step(rng, L, pending, p_term=0.08, p_trunc=0.04):
    x = rng.random(L)
    term = (x < p_term) & ~pending
    trunc = (~term) & (x < p_term + p_trunc) & ~pending
    return term, trunc


def test_acquire_profile_and_dqn_from_the_registry(tmp_path, monkeypatch):
    from ttrl_amd.algos import DQNAgent, check_agent, resolve_and_build
    from ttrl_amd.algos.base import Agent, Transition
    from ttrl_amd.algos.dqn import DQNConfig
    from ttrl_amd.engine import DEFAULT, EngineConfig, acquire
    from ttrl_amd.spaces import ActionSpec, ObsSpec

    monkeypatch.setenv("TTRL_LOCK_DIR", str(tmp_path))
    L, B, A, seed = 2, 16, 6, 11
    cfg = DQNConfig(lr=6.25e-5, adam_eps=1.5e-4, batch_size=B, n_step=3, buffer_capacity=200, train_freq=2,
                    learning_starts=24, target_sync_interval=4)
    spec, aspec = ObsSpec.image(SHAPE), ActionSpec.discrete(A)
    with acquire(0, cfg=DEFAULT) as (device, profile):
        assert profile.gfx == "gfx950", profile
        assert profile.compute_units == 256 and profile.wavefront_size == 64, profile
        assert profile.lds_per_cu == 160 * 1024, profile
        assert profile.hbm_bytes > 250 * 2**30, profile
        agent = resolve_and_build("dqn", spec, aspec, device, cfg=cfg, n_envs=L, seed=seed, profile=profile)
        twin = DQNAgent(spec, aspec, device, cfg=cfg, n_envs=L, seed=seed, engine=EngineConfig())
        try:
            check_agent(agent)
            assert isinstance(agent, Agent) and agent.profile is profile
            for k, v in twin.online.state_dict().items():
                assert np.array_equal(agent.online.state_dict()[k], v), k  # same seeded init
            rng = np.random.default_rng(1)
            obs = rng.integers(0, 256, (L,) + SHAPE, dtype=np.uint8)
            pending = np.zeros(L, bool)
            frame, updates = 0, 0
            for _ in range(60):
                a1, a2 = agent.act(obs), twin.act(obs)
                assert np.array_equal(a1, a2)
                rewards = rng.choice([-1.0, 0.0, 1.0], L, p=[0.1, 0.8, 0.1]).astype(np.float32)
                term, trunc = _env_step(rng, L, pending)
                nxt = rng.integers(0, 256, (L,) + SHAPE, dtype=np.uint8)
                for who in (agent, twin):
                    who.observe(Transition(obs, a1, rewards, term, trunc, nxt))
                pending = term | trunc
                obs = np.where(pending[:, None, None, None], rng.integers(0, 256, (L,) + SHAPE, dtype=np.uint8), nxt)
                frame += L
                due = agent.should_update(frame)
                assert due == twin.should_update(frame)
                if not due:
                    continue
                m, tm = agent.update(), twin.update()
                assert m == tm, (updates, m, tm)
                assert all(np.isfinite(v) for v in m.values()), m
                updates += 1
            assert updates >= 10
            for k, v in twin.online.state_dict().items():
                assert np.array_equal(agent.online.state_dict()[k], v), k
        finally:
            agent.close()
            twin.close()
    assert device.closed


def _acting_oracle(state: dict, frames: np.ndarray, A: int):
    """float64 [logits | value] rows of the shared-trunk actor-critic."""
    from oracle.nets import QNet, qnet_forward
    from oracle.ppo import log_softmax

    items = list(state.items())
    pairs = [(np.asarray(items[i][1], np.float64), np.asarray(items[i + 1][1], np.float64).reshape(-1))
             for i in range(0, len(items), 2)]
    convs = [(w, b, s, 0) for (w, b), s in zip(pairs[:3], (4, 2, 1))]
    (fw, fb), (pw, pb), (vw, vb) = pairs[3:]
    head = (np.concatenate([pw, vw], axis=1), np.concatenate([pb, vb]))
    out, _ = qnet_forward(QNet(convs, [(fw, fb), head], 1.0 / 255.0), frames)
    return log_softmax(out[:, :A]), out[:, A]


def test_ppo_agent_from_the_registry(device):
    from ttrl_amd.algos import check_agent, resolve_and_build
    from ttrl_amd.algos.base import Transition
    from ttrl_amd.algos.ppo import PPOConfig, PPOLearner
    from ttrl_amd.spaces import ActionSpec, ObsSpec
    from ttrl_amd.workloads import he_uniform_qnet_state

    L, A, T, seed = 4, 6, 16, 5
    cfg = PPOConfig(n_steps=T, minibatch_size=32, epochs=2, step_mode="graph")
    spec, aspec = ObsSpec.image(SHAPE), ActionSpec.discrete(A)
    agent = resolve_and_build("ppo", spec, aspec, device, cfg=cfg, n_envs=L, seed=seed)
    twin = PPOLearner(spec, aspec, device, cfg=cfg, seed=seed)
    try:
        check_agent(agent)
        state = he_uniform_qnet_state(agent.net, 9)
        agent.net.load_state_dict(state)
        twin.net.load_state_dict(state)
        mirror = np.random.default_rng(seed)  # the agent's acting generator, replayed on the host
        rng = np.random.default_rng(2)
        obs = rng.integers(0, 256, (L,) + SHAPE, dtype=np.uint8)
        pending = np.zeros(L, bool)
        rows = []
        for step in range(2 * T):
            actions = agent.act(obs)
            rec = agent._pending
            want_logp, want_v = _acting_oracle(agent.net.state_dict(), obs, A)
            got = agent._acting.decide(obs)
            assert float(np.max(np.abs(got["logp"] - want_logp))) <= 1e-4 * max(np.max(np.abs(want_logp)), 1.0)
            assert float(np.max(np.abs(got["value"].reshape(-1) - want_v))) <= 1e-4 * max(np.max(np.abs(want_v)), 1.0)
            probs = np.exp(got["logp"])
            cdf = np.cumsum(probs / probs.sum(-1, keepdims=True), -1)
            want = np.clip((mirror.random(L)[:, None] > cdf).sum(-1), 0, A - 1)
            assert np.array_equal(actions, want), step
            assert np.array_equal(rec["logp"], got["logp"][np.arange(L), actions])
            rewards = rng.choice([-1.0, 0.0, 1.0], L, p=[0.1, 0.8, 0.1]).astype(np.float32)
            term, trunc = _env_step(rng, L, pending)
            nxt = rng.integers(0, 256, (L,) + SHAPE, dtype=np.uint8)
            valid = ~pending
            agent.observe(Transition(obs, actions, rewards, term, trunc, nxt))
            rows.append((obs, actions, rec["logp"], rec["value"], rewards, term.astype(np.float32),
                         valid.astype(np.float32)))
            pending = term | trunc
            obs = np.where(pending[:, None, None, None], rng.integers(0, 256, (L,) + SHAPE, dtype=np.uint8), nxt)
            if not agent.should_update(0):
                assert (step + 1) % T
                continue
            last_v = _acting_oracle(agent.net.state_dict(), nxt, A)[1]
            rollout = {k: np.stack([r[i] for r in rows]) for i, k in
                       enumerate(("obs", "actions", "logp", "values", "rewards", "dones", "valid"))}
            rollout["last_values"] = agent._last_values()
            assert float(np.max(np.abs(rollout["last_values"] - last_v))) <= 1e-4 * max(np.max(np.abs(last_v)), 1.0)
            assert rollout["valid"].min() == 0.0  # padding steps were stored, masked
            m = agent.update()
            tm = twin.update(rollout)
            assert m == tm, (m, tm)
            for k, v in twin.net.state_dict().items():
                assert np.array_equal(agent.net.state_dict()[k], v), k
            rows = []
        assert agent.update_count == 2 and agent.frame_count == 2 * T * L
    finally:
        agent.close()
        twin.close()
