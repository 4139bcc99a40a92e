"""A learner's policy exported to an artifact and run by `load_policy` on the
GPU, against the oracle's float64 restatement of the reference's deployed
forward on the same file (oracle/deploy.py): exact first-index argmax
wherever the top-two gap of the oracle's row exceeds 1e-4 of its scale,
tanh-mapped actions within 2e-5."""

from __future__ import annotations

import numpy as np
import pytest

from tests._dqn_helpers import build_learner
from tests._sac_helpers import build_sac

pytestmark = pytest.mark.gpu


def _decisive(rows: np.ndarray) -> np.ndarray:
    top = np.sort(rows, 1)[:, -2:]
    return (top[:, 1] - top[:, 0]) > 1e-4 * np.abs(rows).max()


def _export(learner, tmp_path, name):
    from ttrl_amd import checkpoint as ck
    from ttrl_amd.deploy import export_policy
    path = str(tmp_path / f"{name}.npz")
    ck.save_checkpoint(path, agent_state=learner.state_dict(weights_only=True), obs_spec=learner.obs_spec,
                       action_spec=learner.action_spec, level=ck.L0)
    return export_policy(path, str(tmp_path / f"{name}.policy.npz"))


def test_dqn_policy_artifact_runs_on_the_device(device, tmp_path):
    from oracle import deploy as odeploy
    from ttrl_amd.deploy import load_policy

    learner, _, _ = build_learner(device, seed=9)
    policy = None
    try:
        art = _export(learner, tmp_path, "dqn")
        meta, arrays = odeploy.read(art)
        policy = load_policy(art, device, lanes=8)
        frames = np.random.default_rng(4).integers(0, 256, (8, 4, 84, 84), dtype=np.uint8)
        got = policy(frames)
        rows = odeploy.head_rows(meta, arrays, frames)
        keep = _decisive(rows)
        assert got.dtype == np.int64 and got.shape == (8,) and keep.sum() >= 4
        assert np.array_equal(got[keep], np.argmax(rows, 1)[keep])
        greedy = learner._acting.decide(frames)["actions"].astype(np.int64)  # the learner's own acting step
        assert np.array_equal(got[keep], greedy[keep])
        one = policy(frames[3])
        assert np.ndim(one) == 0 and int(one) == int(got[3])
    finally:
        if policy is not None:
            policy.close()
        learner.close()


def test_sac_policy_artifact_runs_on_the_device(device, tmp_path):
    from oracle import deploy as odeploy
    from ttrl_amd.deploy import load_policy

    learner, _, _ = build_sac(device, seed=3)
    policy = None
    try:
        art = _export(learner, tmp_path, "sac")
        meta, arrays = odeploy.read(art)
        assert meta["action_map"] == "tanh_bounds"
        policy = load_policy(art, device, lanes=16)
        obs = np.random.default_rng(5).standard_normal((16, 11)).astype(np.float32)
        got = policy(obs)
        want = odeploy.actions(meta, arrays, obs)
        assert got.shape == (16, 3) and np.max(np.abs(got - want)) < 2e-5
        assert np.max(np.abs(policy(obs[5]) - want[5])) < 2e-5
    finally:
        if policy is not None:
            policy.close()
        learner.close()


def test_ppo_policy_artifact_runs_on_the_device(device, tmp_path):
    from oracle import deploy as odeploy
    from ttrl_amd.algos.ppo import PPOConfig, PPOLearner
    from ttrl_amd.deploy import load_policy
    from ttrl_amd.spaces import ActionSpec, ObsSpec
    from ttrl_amd.workloads import he_uniform_qnet_state

    learner = PPOLearner(ObsSpec.image((4, 84, 84)), ActionSpec.discrete(18), device,
                         cfg=PPOConfig(minibatch_size=64, n_steps=32), seed=4)
    policy = None
    try:
        learner.net.load_state_dict(he_uniform_qnet_state(learner.net, 5))
        art = _export(learner, tmp_path, "ppo")
        meta, arrays = odeploy.read(art)
        assert meta["algo"] == "ppo" and meta["action_map"] == "argmax" and meta["n_actions"] == 18
        policy = load_policy(art, device, lanes=4)
        frames = np.random.default_rng(6).integers(0, 256, (4, 4, 84, 84), dtype=np.uint8)
        got = policy(frames)
        rows = odeploy.head_rows(meta, arrays, frames)
        keep = _decisive(rows)
        assert keep.sum() >= 2 and np.array_equal(got[keep], np.argmax(rows, 1)[keep])
    finally:
        if policy is not None:
            policy.close()
        learner.close()


def test_dqn_acting_forward_at_32_lanes_matches_the_deploy_oracle(device, tmp_path):
    """The batch-32 Q-network forward the benchmark times (the learner's
    captured acting graph at 32 lanes over [32, 4, 84, 84] uint8 frames)
    against the oracle's float64 restatement of the reference's numpy deploy
    forward on the exported artifact (ttrl/deploy/artifact.py:188-252): Q at
    rel 1e-4 and the argmax exact on every row whose top-two gap clears the
    reference's decisive band of 1e-3 (tests/hardware/test_deploy_parity.py:281-292).
    Replaying the graph back to back, as the benchmark does, leaves the same
    Q rows."""
    from oracle import deploy as odeploy

    learner, _, _ = build_learner(device, seed=12)
    try:
        assert learner.cfg.batch_size == 32
        art = _export(learner, tmp_path, "dqn32")
        meta, arrays = odeploy.read(art)
        frames = np.random.default_rng(21).integers(0, 256, (32, 4, 84, 84), dtype=np.uint8)
        out = learner._acting.decide(frames)
        rows = odeploy.head_rows(meta, arrays, frames)
        assert out["q"].shape == (32, 6)
        err = np.max(np.abs(out["q"].astype(np.float64) - rows)) / np.max(np.abs(rows))
        assert err < 1e-4, err
        top = np.sort(rows, 1)[:, -2:]
        keep = (top[:, 1] - top[:, 0]) > 1e-3
        assert keep.sum() >= 16
        assert np.array_equal(out["actions"].astype(np.int64)[keep], np.argmax(rows, 1)[keep])
        w = learner._acting._views[32]
        w.graphs[False].replay_n(5)
        device.synchronize()
        assert np.array_equal(w.outs["q"].numpy(), out["q"])
    finally:
        learner.close()
