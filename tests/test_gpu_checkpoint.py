"""Learner state through a checkpoint file on the GPU: a learner restored
from another's L1 file (into its own already-captured update graph) holds
the same parameters, canonical Adam moments, counters and sampling RNG, and
its next update is bit-identical to the original's (same kernels and plans
in one process, as the graph-replay determinism tests rely on).  The
weights-only marker, the config check and a reference-style config record
follow ttrl/algos/checkpoint.py:72-129."""

from __future__ import annotations

import numpy as np
import pytest

from tests._dqn_helpers import build_learner
from tests._sac_helpers import build_sac

pytestmark = pytest.mark.gpu


def _same_tree(a, b, path=""):
    if isinstance(a, dict):
        assert set(a) == set(b), path
        for k in a:
            _same_tree(a[k], b[k], f"{path}.{k}")
    elif isinstance(a, (list, tuple)):
        assert len(a) == len(b), path
        for i, (x, y) in enumerate(zip(a, b)):
            _same_tree(x, y, f"{path}.{i}")
    elif isinstance(a, np.ndarray):
        if a.dtype == np.float64:  # canonical m / v: S * scale then / scale
            assert np.allclose(a, b, rtol=1e-12, atol=0), path
        else:
            assert np.array_equal(a, np.asarray(b)), path
    else:
        assert a == b, path


def test_dqn_state_round_trips_through_a_file(device, tmp_path):
    from ttrl_amd import checkpoint as ck
    from ttrl_amd.workloads import dqn_batch

    a, _, _ = build_learner(device, seed=5)
    b, _, _ = build_learner(device, seed=6)
    try:
        for k in range(2):
            a.update(dqn_batch(300 + k))
        a.act(np.random.default_rng(0).integers(0, 256, (1, 4, 84, 84), dtype=np.uint8))
        b.update(dqn_batch(999))  # b's graph is captured before the restore
        path = str(tmp_path / "dqn.npz")
        ck.save_checkpoint(path, agent_state=a.state_dict(), obs_spec=a.obs_spec, action_spec=a.action_spec,
                           level=ck.L1, config=a.cfg, frame=a.frame_count)
        loaded = ck.load_checkpoint(path)
        assert loaded["config"] == a.cfg and loaded["frame"] == a.frame_count
        # the names the reference's exporter reads (ttrl/deploy/policies.py:91-97)
        assert {"encoder.towers.obs.layers.0.weight", "encoder.towers.obs.layers.7.weight",
                "head.q.weight"} <= set(loaded["agent_state"]["online"])
        online = loaded["agent_state"]["online"]
        assert online["encoder.towers.obs.layers.0.weight"].shape == (32, 4, 8, 8)  # logical OIHW
        assert online["encoder.towers.obs.layers.7.weight"].shape == (3136, 512)  # (in, out)
        b.load_state_dict(loaded["agent_state"])
        _same_tree(a.state_dict(), b.state_dict())
        ma, mb = a.update(dqn_batch(302)), b.update(dqn_batch(302))
        assert ma["loss"] == mb["loss"] and ma["mean_q"] == mb["mean_q"]
        for k, v in a.online.state_dict().items():
            assert np.array_equal(v, b.online.state_dict()[k]), k
        assert a.update_count == b.update_count
        assert a._rng.random() == b._rng.random()

        weights = a.state_dict(weights_only=True)
        assert weights["weights_only"] is True and "optimizer" not in weights
        with pytest.raises(ValueError, match="parameters only"):
            b.load_state_dict(weights)
        b.load_state_dict(weights, weights_only=True)

        foreign = a.state_dict()
        # a reference config whose mapped fields agree loads (its dispatch mode and
        # its unmapped fields are carried); one that differs in a mapped field does not
        foreign["config"] = ck.StoredDataclass("ttrl.algos.dqn.config:DQNConfig", {
            "double": True, "gamma": a.cfg.gamma, "lr": a.cfg.lr, "step_mode": "traced_fwd_bwd",
            "train_freq": 4, "priority": {"alpha": 0.6}})
        b.load_state_dict(foreign)
        for field, value in (("gamma", 0.5), ("n_step", 5), ("target_sync_interval", 10), ("priority", None)):
            changed = a.state_dict()
            changed["config"] = ck.StoredDataclass("ttrl.algos.dqn.config:DQNConfig", {"double": True, field: value})
            with pytest.raises(ValueError, match="configuration differs"):
                b.load_state_dict(changed)
        other = a.state_dict()
        other["config"] = type(a.cfg)(lr=1e-3)
        with pytest.raises(ValueError, match="configuration differs"):
            b.load_state_dict(other)
        broken = a.state_dict()
        del broken["optimizer"]
        with pytest.raises(ValueError, match="missing"):
            b.load_state_dict(broken)
    finally:
        a.close()
        b.close()


def test_sac_state_round_trips_through_a_file(device, tmp_path):
    from ttrl_amd import checkpoint as ck
    from ttrl_amd.workloads import sac_batch

    a, _, _ = build_sac(device, seed=7)
    b, _, _ = build_sac(device, seed=8)
    try:
        for k in range(2):
            a.update(sac_batch(70 + k))
        b.update(sac_batch(99))
        b.update(sac_batch(98))  # b's update graph is captured before the restore
        path = str(tmp_path / "sac.npz")
        ck.save_checkpoint(path, agent_state=a.state_dict(), obs_spec=a.obs_spec, action_spec=a.action_spec,
                           level=ck.L0)
        loaded = ck.load_checkpoint(path)
        assert loaded["level"] == ck.L0 and loaded["action_spec"].dim == 3
        assert {"policy.encoder.towers.obs.layers.0.weight", "policy.head.heads.mean.weight",
                "critics.0.head.layers.0.weight"} <= set(loaded["agent_state"]["nets"])  # policies.py:69-77
        b.load_state_dict(loaded["agent_state"])
        _same_tree(a.state_dict(), b.state_dict())
        ma, mb = a.update(sac_batch(72)), b.update(sac_batch(72))
        assert ma["critic_loss"] == mb["critic_loss"] and ma["actor_loss"] == mb["actor_loss"]
        for k, v in a.nets.state_dict().items():
            assert np.array_equal(v, b.nets.state_dict()[k]), k
        assert np.array_equal(a.log_alpha.numpy(), b.log_alpha.numpy())
    finally:
        a.close()
        b.close()


def test_ppo_state_round_trips_through_a_file(device, tmp_path):
    from ttrl_amd import checkpoint as ck
    from ttrl_amd.algos.ppo import PPOConfig, PPOLearner
    from ttrl_amd.spaces import ActionSpec, ObsSpec
    from ttrl_amd.workloads import he_uniform_qnet_state, ppo_rollout

    cfg = PPOConfig(minibatch_size=64, epochs=2, n_steps=32)
    learners = []
    for seed in (11, 12):
        lr = PPOLearner(ObsSpec.image((4, 84, 84)), ActionSpec.discrete(6), device, cfg=cfg, seed=seed)
        lr.net.load_state_dict(he_uniform_qnet_state(lr.net, seed + 1))
        learners.append(lr)
    a, b = learners
    try:
        a.update(ppo_rollout(20, 32, 4, 6))
        b.update(ppo_rollout(21, 32, 4, 6))  # b's minibatch graph is captured before the restore
        path = str(tmp_path / "ppo.npz")
        ck.save_checkpoint(path, agent_state=a.state_dict(), obs_spec=a.obs_spec, action_spec=a.action_spec,
                           level=ck.L1, config=a.cfg, frame=a.frame_count)
        agent_state = ck.load_checkpoint(path)["agent_state"]
        assert {"encoders.actor.towers.obs.layers.0.weight",
                "heads.policy.logits.weight"} <= set(agent_state["net"])  # policies.py:78-90
        b.load_state_dict(agent_state)
        _same_tree(a.state_dict(), b.state_dict())
        rollout = ppo_rollout(22, 32, 4, 6)
        ma, mb = a.update(rollout), b.update(rollout)
        for k in PPOLearner.METRICS:
            assert ma[k] == mb[k], k
        for k, v in a.net.state_dict().items():
            assert np.array_equal(v, b.net.state_dict()[k]), k
    finally:
        a.close()
        b.close()


def test_recurrent_ppo_state_round_trips_through_a_file(device, tmp_path):
    """The GRU memories keep the reference's names (`memories.<role>.cell.*`)
    while the conv tower moves under `encoders.<role>.towers.obs`."""
    from ttrl_amd import checkpoint as ck
    from ttrl_amd.algos.ppo import PPOConfig, RecurrentConfig, RecurrentPPOLearner
    from ttrl_amd.spaces import ActionSpec, ObsSpec
    from ttrl_amd.workloads import he_uniform_qnet_state, recurrent_ppo_rollout

    T, N, L, Hd, mb, A = 16, 4, 8, 32, 16, 6
    cfg = PPOConfig(minibatch_size=mb, epochs=2, n_steps=T, recurrent=RecurrentConfig(hidden_size=Hd, seq_len=L))
    learners = []
    for seed in (51, 52):
        lr = RecurrentPPOLearner(ObsSpec.image((4, 84, 84)), ActionSpec.discrete(A), device, cfg=cfg, seed=seed)
        lr.net.load_state_dict(he_uniform_qnet_state(lr.net, seed + 1))
        learners.append(lr)
    a, b = learners
    try:
        a.update(recurrent_ppo_rollout(60, T, N, A, L, Hd))
        b.update(recurrent_ppo_rollout(61, T, N, A, L, Hd))
        path = str(tmp_path / "rppo.npz")
        ck.save_checkpoint(path, agent_state=a.state_dict(), obs_spec=a.obs_spec, action_spec=a.action_spec,
                           level=ck.L1, config=a.cfg, frame=a.frame_count)
        agent_state = ck.load_checkpoint(path)["agent_state"]
        names = set(agent_state["net"])
        assert "encoders.actor.towers.obs.layers.0.weight" in names
        assert any(k.startswith("memories.actor.cell.") for k in names) and not any("towers" in k and "memories" in k
                                                                                  for k in names)
        b.load_state_dict(agent_state)
        _same_tree(a.state_dict(), b.state_dict())
        rollout = recurrent_ppo_rollout(62, T, N, A, L, Hd)
        ma, mb_ = a.update(rollout), b.update(rollout)
        for k in RecurrentPPOLearner.METRICS:
            assert ma[k] == mb_[k], k
        for k, v in a.net.state_dict().items():
            assert np.array_equal(v, b.net.state_dict()[k]), k
        with pytest.raises(ValueError, match="configuration differs"):
            other = a.state_dict()
            other["config"] = PPOConfig()
            b.load_state_dict(other)
    finally:
        a.close()
        b.close()
