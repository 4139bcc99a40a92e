"""Policy artifact export (ttrl_amd/deploy.py) on the CPU, and the pins of the
deployed-forward oracle (oracle/deploy.py).

The artifact's members and meta are the reference exporter's
(ttrl/deploy/export.py:77-180): conv stages in OIHW with the observation
scale folded into the first, a vector trunk's first Linear scaled instead,
trunk and head pairs, bounds for a bounded map, the format marker and the
conv geometry.  The oracle's conv path is checked against
oracle/nets.qnet_forward on the same weights (that forward is pinned
against torch's conv2d), and its action maps against their closed forms."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import deploy as odeploy
from ttrl_amd import checkpoint as ck
from ttrl_amd import deploy
from ttrl_amd.spaces import ActionSpec, ObsSpec


def _dqn_online(rng, A=6):
    shapes = [((32, 4, 8, 8), 32), ((64, 32, 4, 4), 64), ((64, 64, 3, 3), 64)]
    state = {}
    for (shape, out), index in zip(shapes, (0, 2, 4)):
        fan = np.prod(shape[1:])
        state[f"encoder.towers.obs.layers.{index}.weight"] = (rng.standard_normal(shape) / np.sqrt(fan)).astype(np.float32)
        state[f"encoder.towers.obs.layers.{index}.bias"] = (0.1 * rng.standard_normal(out)).astype(np.float32)
    state["encoder.towers.obs.layers.7.weight"] = (rng.standard_normal((3136, 512)) / 56).astype(np.float32)
    state["encoder.towers.obs.layers.7.bias"] = (0.1 * rng.standard_normal((1, 512))).astype(np.float32)
    state["head.q.weight"] = (rng.standard_normal((512, A)) / 22).astype(np.float32)
    state["head.q.bias"] = (0.1 * rng.standard_normal((1, A))).astype(np.float32)
    return state


def _dqn_checkpoint(tmp_path, rng):
    from ttrl_amd.algos.dqn import DQNConfig
    online = _dqn_online(rng)
    path = str(tmp_path / "dqn.npz")
    ck.save_checkpoint(path, agent_state={"online": online, "target": online, "config": DQNConfig()},
                       obs_spec=ObsSpec.image((4, 84, 84)), action_spec=ActionSpec.discrete(6), level=ck.L0)
    return path, online


def test_dqn_export_members_meta_and_forward(tmp_path):
    from oracle.nets import QNet, qnet_forward
    rng = np.random.default_rng(0)
    ckpt, online = _dqn_checkpoint(tmp_path, rng)
    out = deploy.export_policy(ckpt, str(tmp_path / "dqn.policy.npz"))
    meta, arrays = deploy.read_artifact(out)
    assert set(arrays) == {"conv.0.weight", "conv.0.bias", "conv.1.weight", "conv.1.bias", "conv.2.weight",
                           "conv.2.bias", "trunk.0.weight", "trunk.0.bias", "head.weight", "head.bias"}
    assert meta["artifact_format"] == "ttrl-policy-9c2e57" and meta["algo"] == "dqn"
    assert meta["action_map"] == "argmax" and meta["action_kind"] == "discrete" and meta["n_actions"] == 6
    assert meta["obs_dim"] is None and meta["obs_shape"] == [4, 84, 84] and meta["trunk_layers"] == 1
    assert meta["conv"] == [{"stride": 4, "padding": 0}, {"stride": 2, "padding": 0}, {"stride": 1, "padding": 0}]
    assert meta["action_dim"] is None and meta["action_mask"] == 0 and meta["normalizer"] is None
    w0 = online["encoder.towers.obs.layers.0.weight"]
    assert np.array_equal(arrays["conv.0.weight"], w0 * np.float32(1.0 / 255.0))
    assert np.array_equal(arrays["conv.1.weight"], online["encoder.towers.obs.layers.2.weight"])
    assert np.array_equal(arrays["trunk.0.weight"], online["encoder.towers.obs.layers.7.weight"])
    assert arrays["trunk.0.bias"].shape == (512,) and arrays["head.bias"].shape == (6,)
    # the oracle's deployed forward against the pinned Q-network oracle on the
    # unfolded weights: the same rows, so the same decisive actions
    convs = [(online[f"encoder.towers.obs.layers.{i}.weight"].astype(np.float64),
              online[f"encoder.towers.obs.layers.{i}.bias"].astype(np.float64), s, 0)
             for i, s in zip((0, 2, 4), (4, 2, 1))]
    fcs = [(online["encoder.towers.obs.layers.7.weight"].astype(np.float64),
            online["encoder.towers.obs.layers.7.bias"].astype(np.float64).reshape(-1)),
           (online["head.q.weight"].astype(np.float64), online["head.q.bias"].astype(np.float64).reshape(-1))]
    frames = rng.integers(0, 256, (5, 4, 84, 84), dtype=np.uint8)
    q, _ = qnet_forward(QNet(convs, fcs, 1.0 / 255.0), frames)
    rows = odeploy.head_rows(meta, arrays, frames)
    assert np.max(np.abs(rows - q)) <= 1e-6 * np.abs(q).max()
    assert np.array_equal(odeploy.actions(meta, arrays, frames), np.argmax(q, 1))


def test_sac_export_folds_the_vector_scale_and_maps_through_tanh(tmp_path):
    from ttrl_amd.algos.sac import SACConfig
    rng = np.random.default_rng(1)
    nets = {"policy.encoder.towers.obs.layers.0.weight": rng.standard_normal((11, 64)).astype(np.float32),
            "policy.encoder.towers.obs.layers.0.bias": rng.standard_normal((1, 64)).astype(np.float32),
            "policy.encoder.towers.obs.layers.2.weight": (rng.standard_normal((64, 64)) / 8).astype(np.float32),
            "policy.encoder.towers.obs.layers.2.bias": rng.standard_normal((1, 64)).astype(np.float32),
            "policy.head.heads.mean.weight": (rng.standard_normal((64, 3)) / 8).astype(np.float32),
            "policy.head.heads.mean.bias": rng.standard_normal((1, 3)).astype(np.float32),
            "policy.head.heads.log_std.weight": np.zeros((64, 3), np.float32),
            "policy.head.heads.log_std.bias": np.zeros((1, 3), np.float32),
            "critics.0.head.layers.0.weight": np.zeros((14, 8), np.float32)}
    spec = ObsSpec.vector(11, scale=0.5)
    act = ActionSpec.continuous(3, (-1.0, 0.0, -2.0), (1.0, 4.0, 2.0))
    path = str(tmp_path / "sac.npz")
    ck.save_checkpoint(path, agent_state={"nets": nets, "log_alpha": np.zeros((1, 1), np.float32),
                                          "config": SACConfig()}, obs_spec=spec, action_spec=act, level=ck.L0)
    meta, arrays = deploy.read_artifact(deploy.export_policy(path, str(tmp_path / "sac.policy.npz")))
    assert meta["algo"] == "sac" and meta["action_map"] == "tanh_bounds" and meta["obs_dim"] == 11
    assert meta["conv"] == [] and meta["trunk_layers"] == 2 and meta["action_dim"] == 3 and meta["n_actions"] is None
    assert np.array_equal(arrays["trunk.0.weight"], nets["policy.encoder.towers.obs.layers.0.weight"] * np.float32(0.5))
    assert np.array_equal(arrays["action_low"], act.low_array) and np.array_equal(arrays["action_high"], act.high_array)
    obs = rng.standard_normal((7, 11)).astype(np.float32)
    h = np.maximum((obs.astype(np.float64) * 0.5) @ nets["policy.encoder.towers.obs.layers.0.weight"]
                   + nets["policy.encoder.towers.obs.layers.0.bias"], 0)
    h = np.maximum(h @ nets["policy.encoder.towers.obs.layers.2.weight"] + nets["policy.encoder.towers.obs.layers.2.bias"], 0)
    mean = h @ nets["policy.head.heads.mean.weight"] + nets["policy.head.heads.mean.bias"]
    want = np.array([0.0, 2.0, 0.0]) + np.array([1.0, 2.0, 2.0]) * np.tanh(mean)
    assert np.allclose(odeploy.actions(meta, arrays, obs), want, rtol=1e-6, atol=1e-6)
    meta_clip = dict(meta, action_map="clip_bounds")
    assert np.allclose(odeploy.actions(meta_clip, arrays, obs), np.clip(mean, act.low_array, act.high_array),
                       rtol=1e-6, atol=1e-6)


def test_refusals(tmp_path):
    from ttrl_amd.algos.ppo import PPOConfig
    rng = np.random.default_rng(2)
    ckpt, online = _dqn_checkpoint(tmp_path, rng)
    with pytest.raises(ValueError, match="CHECKPOINT"):
        deploy.read_artifact(ckpt)
    out = deploy.export_policy(ckpt, str(tmp_path / "p.npz"))
    meta, arrays = deploy.read_artifact(out)
    import json
    bad = dict(arrays)
    bad["__meta__"] = np.frombuffer(json.dumps(dict(meta, artifact_format="ttrl-policy-000000")).encode(), np.uint8)
    np.savez(tmp_path / "bad.npz", **bad)
    with pytest.raises(ValueError, match="artifact marker"):
        deploy.read_artifact(str(tmp_path / "bad.npz"))
    # a recurrent PPO policy has no feedforward artifact
    net = {"encoders.actor.towers.obs.layers.0.weight": np.zeros((4, 8), np.float32),
           "encoders.actor.towers.obs.layers.0.bias": np.zeros(8, np.float32),
           "memories.actor.cell.weight_ih": np.zeros((8, 24), np.float32),
           "heads.policy.logits.weight": np.zeros((8, 2), np.float32),
           "heads.policy.logits.bias": np.zeros(2, np.float32)}
    path = str(tmp_path / "rppo.npz")
    ck.save_checkpoint(path, agent_state={"net": net, "config": PPOConfig()}, obs_spec=ObsSpec.vector(4),
                       action_spec=ActionSpec.discrete(2), level=ck.L0)
    with pytest.raises(ValueError, match="recurrent"):
        deploy.export_policy(path, str(tmp_path / "x.npz"))
    # a config no source names
    path = str(tmp_path / "other.npz")
    ck.save_checkpoint(path, agent_state={"net": net, "config": ck.StoredDataclass("ttrl.algos.x:XConfig", {})},
                       obs_spec=ObsSpec.vector(4), action_spec=ActionSpec.discrete(2), level=ck.L0)
    with pytest.raises(ValueError, match="XConfig"):
        deploy.export_policy(path, str(tmp_path / "y.npz"))


def test_a_reference_config_record_selects_its_source(tmp_path):
    rng = np.random.default_rng(3)
    online = _dqn_online(rng)
    path = str(tmp_path / "ref.npz")
    cfg = ck.StoredDataclass("ttrl.algos.dqn.config:DQNConfig", {"encoder": "auto"})
    ck.save_checkpoint(path, agent_state={"online": online, "config": cfg}, obs_spec=ObsSpec.image((4, 84, 84)),
                       action_spec=ActionSpec.discrete(6), level=ck.L0)
    meta, _ = deploy.read_artifact(deploy.export_policy(path, str(tmp_path / "ref.policy.npz")))
    assert meta["algo"] == "dqn"
