"""The GPU-resident replay against the replay oracle (oracle/replay.py), both
driven with the same writes and seeds: every sampled batch must be the
oracle's -- the same (lane, column) draws (the generator is consumed on the
host in the reference's order), bit-identical observations, successors,
actions, float32 returns, dones and discounts -- and the importance-sampling
weights within rel 1e-6 (float64 powers on the device against numpy's).
Lanes, ring wrap-around, episode boundaries with their final observations,
uniform and prioritized draws, priority updates from the host and from the
device, and a batch assembled straight into a DQN learner's bound inputs
(ttrl/buffers/replay.py, ttrl/buffers/sampling.py, ttrl/buffers/indexing.py).
"""

from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _pair(device, spec, *, capacity, n_envs, n_step, gamma, seed, priority=None, boundary_rows=None):
    from oracle.replay import ReplayOracle
    from ttrl_amd.buffers import ReplayBuffer
    from ttrl_amd.spaces import ActionSpec

    buf = ReplayBuffer(spec, ActionSpec.discrete(5), device, capacity=capacity, n_envs=n_envs, n_step=n_step,
                       gamma=gamma, seed=seed, priority=priority, boundary_rows=boundary_rows)
    shape = tuple(spec.shape) if spec.kind == "image" else (spec.size,)
    dtype = np.uint8 if spec.kind == "image" else np.float32
    orc = ReplayOracle(shape, dtype, capacity=capacity, n_envs=n_envs, n_step=n_step, gamma=gamma, seed=seed,
                       alpha=None if priority is None else priority.alpha,
                       epsilon=1e-6 if priority is None else priority.epsilon)
    return buf, orc, shape, dtype


def _step(buf, orc, rng, shape, dtype, p_end=0.15):
    L = buf.n_envs
    if dtype == np.uint8:
        obs = rng.integers(0, 256, (L,) + shape, dtype=np.uint8)
    else:
        obs = rng.standard_normal((L,) + shape).astype(np.float32)
    actions = rng.integers(0, 5, L)
    rewards = rng.standard_normal(L).astype(np.float32)
    x = rng.random(L)
    term = x < 0.6 * p_end
    trunc = (~term) & (x < p_end)
    ended = term | trunc
    final = [None] * L
    for lane in np.flatnonzero(ended):
        final[lane] = (rng.integers(0, 256, shape, dtype=np.uint8) if dtype == np.uint8
                       else rng.standard_normal(shape).astype(np.float32))
    buf.add_batch(obs, actions, rewards, term, trunc, final)
    orc.add_batch(obs, actions, rewards, term, trunc, final)


def _same(got: dict, want: dict, weights_rel=1e-6):
    for k in ("lanes", "cols"):
        assert np.array_equal(got[k].reshape(-1), np.asarray(want[k]).reshape(-1)), k
    assert np.array_equal(got["obs"], want["obs"])
    assert np.array_equal(got["next_obs"], want["next_obs"])
    assert np.array_equal(got["actions"].reshape(-1), want["actions"].reshape(-1))
    for k in ("rewards", "dones", "discounts"):
        assert np.array_equal(got[k].reshape(-1), want[k].reshape(-1)), k
    if want["weights"] is None:
        assert got["weights"] is None
    else:
        w = np.asarray(want["weights"], np.float64)
        assert np.max(np.abs(got["weights"].reshape(-1) - w)) <= weights_rel * w.max()


@pytest.mark.parametrize("kind", ["vector", "image"])
def test_uniform_batches_match_the_oracle(device, kind):
    from ttrl_amd.spaces import ObsSpec

    spec = ObsSpec.vector(3) if kind == "vector" else ObsSpec.image((4, 84, 84))
    buf, orc, shape, dtype = _pair(device, spec, capacity=96, n_envs=3, n_step=3, gamma=0.9, seed=7)
    rng = np.random.default_rng(1)
    for _ in range(3):  # pos 3 = n_step: nothing sampleable yet
        _step(buf, orc, rng, shape, dtype)
    with pytest.raises(ValueError, match="no lane holds"):
        buf.sample(4)
    for round_ in range(6):
        for _ in range(9):  # 54 steps in all: every lane wraps its 32 columns
            _step(buf, orc, rng, shape, dtype)
        assert buf.num_sampleable == int(orc.sampleable()[1].sum())
        _same(buf.sample(32).host(), orc.sample(32))
    assert buf.num_boundaries == len(orc.final) > 0
    with pytest.raises(ValueError, match="samples uniformly"):
        buf.sample(8, beta=0.4)


def test_prioritized_batches_and_updates_match_the_oracle(device):
    from ttrl_amd.buffers import PriorityConfig
    from ttrl_amd.engine.tensor import DeviceArray
    from ttrl_amd.spaces import ObsSpec

    cfg = PriorityConfig(alpha=0.6)
    buf, orc, shape, dtype = _pair(device, ObsSpec.vector(2), capacity=2500, n_envs=2, n_step=3, gamma=0.99,
                                   seed=11, priority=cfg)
    rng = np.random.default_rng(2)
    for _ in range(1400):  # each lane wraps its 1250 columns; two chunks of the pick per lane
        _step(buf, orc, rng, shape, dtype, p_end=0.01)
    for round_ in range(4):
        got = buf.sample(64, beta=0.4 + 0.1 * round_)
        want = orc.sample(64, beta=0.4 + 0.1 * round_)
        _same(got.host(), want)
        td = rng.uniform(0.0, 5.0, 64)
        if round_ % 2:
            buf.update_priorities(want["lanes"], want["cols"], td)  # float64 end to end
        else:
            td = td.astype(np.float32)  # TD errors an update left on the device
            dev_td = DeviceArray(device, (64,), np.float32)
            dev_td.upload(td)
            buf.update_priorities_device(got, dev_td)
        orc.update_priorities(want["lanes"], want["cols"], td)
        table = buf.priorities_numpy()
        assert np.max(np.abs(table - orc.weight)) <= 1e-12 * orc.weight.max()
        for _ in range(5):
            _step(buf, orc, rng, shape, dtype, p_end=0.01)
    with pytest.raises(ValueError, match="need a beta"):
        buf.sample(8)
    with pytest.raises(ValueError, match="NaN or infinite"):
        buf.update_priorities([0], [0], [np.nan])
    # a non-finite TD error from the device path is caught by the next draw
    got = buf.sample(8, beta=0.5)
    bad = DeviceArray(device, (8,), np.float32)
    bad.upload(np.array([1.0, np.nan, 2.0, 3.0, 1.0, 1.0, 1.0, 1.0], np.float32))
    buf.update_priorities_device(got, bad)
    with pytest.raises(ValueError, match="NaN or infinite"):
        buf.sample(8, beta=0.5)


def test_a_batch_lands_in_the_learner_inputs(device):
    """Sampling into a DQN learner's bound inputs gives the update the
    oracle's batch: the update's metrics equal those of the same batch
    loaded from the host."""
    from ttrl_amd.algos.dqn import DQNConfig, DQNLearner, leaf_key
    from ttrl_amd.buffers import PriorityConfig
    from ttrl_amd.spaces import ActionSpec, ObsSpec
    from ttrl_amd.workloads import he_uniform_qnet_state

    spec = ObsSpec.image((4, 84, 84))
    buf, orc, shape, dtype = _pair(device, spec, capacity=400, n_envs=4, n_step=3, gamma=0.99, seed=13,
                                   priority=PriorityConfig())
    rng = np.random.default_rng(3)
    for _ in range(40):
        _step(buf, orc, rng, shape, dtype, p_end=0.05)
    learners = []
    for _ in range(2):
        lr = DQNLearner(spec, ActionSpec.discrete(5), device,
                        cfg=DQNConfig(batch_size=32, step_mode="eager", prioritized=True), seed=1)
        lr.online.load_state_dict(he_uniform_qnet_state(lr.online, 2))
        lr.target.copy_from(lr.online)
        learners.append(lr)
    try:
        ins = learners[0].inputs
        out = {"obs": ins[leaf_key("obs", spec.name)].data, "next_obs": ins[leaf_key("next_obs", spec.name)].data,
               "actions_onehot": ins["actions_onehot"].data, "rewards": ins["rewards"].data,
               "dones": ins["dones"].data, "discounts": ins["discounts"].data, "weights": ins["is_weights"].data}
        buf.sample(32, beta=0.4, out=out)
        m0 = learners[0].update()
        want = orc.sample(32, beta=0.4)
        m1 = learners[1].update({"obs": want["obs"], "next_obs": want["next_obs"], "actions": want["actions"],
                                 "rewards": want["rewards"], "dones": want["dones"],
                                 "discounts": want["discounts"], "is_weights": want["weights"]})
        assert m0["loss"] == pytest.approx(m1["loss"], rel=1e-6)
        assert m0["mean_q"] == pytest.approx(m1["mean_q"], rel=1e-6)
        assert np.allclose(m0["td_abs"], m1["td_abs"], rtol=1e-6, atol=1e-7)
    finally:
        for lr in learners:
            lr.close()


def test_bulk_steps_equal_successive_steps(device):
    """add_steps(T steps) writes what T add_batch calls write, boundaries
    included."""
    from ttrl_amd.spaces import ObsSpec

    spec = ObsSpec.image((2, 6, 6))
    buf, orc, shape, dtype = _pair(device, spec, capacity=60, n_envs=3, n_step=2, gamma=0.95, seed=17)
    rng = np.random.default_rng(4)
    T, L = 33, 3
    obs = rng.integers(0, 256, (T, L) + shape, dtype=np.uint8)
    actions = rng.integers(0, 5, (T, L))
    rewards = rng.standard_normal((T, L)).astype(np.float32)
    x = rng.random((T, L))
    term, trunc = x < 0.1, (x >= 0.1) & (x < 0.2)
    final = rng.integers(0, 256, (T, L) + shape, dtype=np.uint8)
    buf.add_steps(obs[:20], actions[:20], rewards[:20], term[:20], trunc[:20], final[:20])
    buf.add_steps(obs[20:], actions[20:], rewards[20:], term[20:], trunc[20:], final[20:])
    for t in range(T):
        ended = term[t] | trunc[t]
        orc.add_batch(obs[t], actions[t], rewards[t], term[t], trunc[t],
                      [final[t, l] if ended[l] else None for l in range(L)])
    assert buf.num_boundaries == len(orc.final)
    for _ in range(3):
        _same(buf.sample(24).host(), orc.sample(24))
