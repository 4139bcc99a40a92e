"""The checkpoint container (ttrl_amd/checkpoint.py) on the CPU, against the
behaviour the reference's own checkpoint tests fix
(tests/train/test_checkpoint_bytes.py, test_checkpoint.py,
test_checkpoint_contract.py): byte-exact blobs under their own marker, the
format marker checked for equality, the level rules, members under
`state.<path>`, and the specs' stored forms with the reference's field
names (ttrl/spaces/obs.py:82-130, ttrl/spaces/action.py:34-39,
ttrl/train/checkpoint/specs.py:31-62)."""

from __future__ import annotations

import json
import sys

import numpy as np
import pytest

from ttrl_amd import checkpoint as ck
from ttrl_amd.algos.dqn import DQNConfig
from ttrl_amd.spaces import ActionSpec, ObsSpec


def _save(path, **kw):
    args = {"agent_state": {"w": np.zeros(2, np.float32)}, "obs_spec": ObsSpec.vector(2),
            "action_spec": ActionSpec.discrete(2), "level": ck.L0}
    args.update(kw)
    ck.save_checkpoint(str(path), **args)
    return str(path)


def test_tree_round_trip_keeps_types_and_values(tmp_path):
    blob = bytes(range(256)) * 7 + b"\x00\xff trailing"
    state = {"online": {"conv1.weight": np.arange(24, dtype=np.float32).reshape(2, 3, 2, 2),
                        "frames": np.arange(6, dtype=np.uint8)},
             "optimizer": {"t": 3, "steps": [3, 3], "betas": (0.9, 0.999), "m": [np.ones(4), np.zeros(2)]},
             "rng": blob, "count": np.int64(7), "note": None, "flag": True, "config": DQNConfig(lr=1e-4)}
    path = _save(tmp_path / "c.npz", agent_state=state)
    back = ck.load_checkpoint(path)["agent_state"]
    assert type(back["rng"]) is bytes and back["rng"] == blob
    assert np.array_equal(back["online"]["conv1.weight"], state["online"]["conv1.weight"])
    assert back["online"]["frames"].dtype == np.uint8
    assert back["optimizer"]["steps"] == [3, 3] and back["optimizer"]["betas"] == [0.9, 0.999]
    assert back["count"] == 7 and type(back["count"]) is int
    assert back["note"] is None and back["flag"] is True
    assert back["config"] == DQNConfig(lr=1e-4)
    arrays, meta = ck.read_meta(path)
    assert meta["agent_state"]["rng"] == {"__bytes__": "state.rng"}
    assert meta["agent_state"]["online"]["conv1.weight"] == {"__array__": "state.online.conv1.weight"}
    assert meta["agent_state"]["optimizer"]["m"] == {"__list__": [{"__array__": "state.optimizer.m.0"},
                                                                 {"__array__": "state.optimizer.m.1"}]}
    assert meta["agent_state"]["config"]["__dataclass__"] == "ttrl_amd.algos.dqn:DQNConfig"
    assert set(arrays) == {"state.online.conv1.weight", "state.online.frames", "state.rng",
                           "state.optimizer.m.0", "state.optimizer.m.1"}


def test_foreign_dataclass_comes_back_as_a_record_and_is_never_imported(tmp_path):
    rec = ck.StoredDataclass("ttrl.algos.dqn.config:DQNConfig", {"gamma": 0.99, "double": True})
    path = _save(tmp_path / "c.npz", agent_state={"config": rec, "w": np.ones(3, np.float32)})
    assert "ttrl" not in sys.modules
    back = ck.load_checkpoint(path)["agent_state"]["config"]
    assert back == rec and "ttrl" not in sys.modules
    # and writes back out unchanged
    path2 = _save(tmp_path / "d.npz", agent_state={"config": back})
    assert ck.read_meta(path2)[1]["agent_state"]["config"] == {
        "__dataclass__": "ttrl.algos.dqn.config:DQNConfig", "fields": {"gamma": 0.99, "double": True}}


def test_unknown_or_missing_fields_of_own_dataclasses_are_named(tmp_path):
    path = _save(tmp_path / "c.npz", agent_state={"config": DQNConfig()})
    arrays, meta = ck.read_meta(path)
    meta["agent_state"]["config"]["fields"]["renamed_field"] = 1
    with pytest.raises(ck.CheckpointFieldError, match="renamed_field"):
        ck.join(meta["agent_state"], arrays, file=path)
    for bad in ("ttrl_amd.no_such_module:X", "ttrl_amd.algos.dqn:NoSuchClass", "ttrl_amd.algos.dqn:DQNLearner.act"):
        with pytest.raises(ck.CheckpointFieldError, match="not a dataclass"):
            ck.join({"__dataclass__": bad, "fields": {}}, arrays, file=path)


def test_format_marker_and_unreadable_files_are_refused(tmp_path):
    path = _save(tmp_path / "c.npz")
    arrays, meta = ck.read_meta(path)
    meta["format"] = "ttrl-checkpoint-000000"
    bad = tmp_path / "bad.npz"
    np.savez(bad, **arrays, __meta__=np.frombuffer(json.dumps(meta).encode(), np.uint8))
    with pytest.raises(ValueError, match="format marker"):
        ck.load_checkpoint(str(bad))
    junk = tmp_path / "junk.npz"
    junk.write_bytes(b"not a zip")
    with pytest.raises(ValueError, match="not a readable ttrl checkpoint"):
        ck.read_meta(str(junk))
    assert meta["format"] != ck.FORMAT == "ttrl-checkpoint-9c42ad"


def test_level_rules(tmp_path):
    with pytest.raises(ValueError, match="level must be one of"):
        _save(tmp_path / "a.npz", level="L2")
    with pytest.raises(ValueError, match="replay_state"):
        _save(tmp_path / "b.npz", replay_state={"obs": np.zeros(3)})
    with pytest.raises(ValueError, match="cadence_state"):
        _save(tmp_path / "c.npz", cadence_state={"n": 1})
    with pytest.raises(ValueError, match="config"):
        _save(tmp_path / "d.npz", level=ck.L1)
    path = _save(tmp_path / "e.npz", level=ck.L1, config=DQNConfig(), frame=1234, replay_state={"pos": 5})
    out = ck.load_checkpoint(path)
    assert out["level"] == ck.L1 and out["frame"] == 1234 and out["config"] == DQNConfig()
    assert out["replay_state"] == {"pos": 5} and out["env_reward_state"] is None and out["cadence_state"] is None
    l0 = ck.load_checkpoint(_save(tmp_path / "f.npz"))
    assert "frame" not in l0 and l0["env_policy_state"] is None and l0["extra"] == {}


def test_non_string_keys_and_unknown_leaf_types_are_refused(tmp_path):
    with pytest.raises(TypeError, match="non-string keys"):
        _save(tmp_path / "a.npz", agent_state={1: np.zeros(1)})
    with pytest.raises(TypeError, match="no JSON or array"):
        _save(tmp_path / "b.npz", agent_state={"x": object()})


def test_spec_forms_carry_the_reference_field_names(tmp_path):
    obs = ObsSpec.image((4, 84, 84))
    stored = ck.obs_spec_to_json(obs)
    leaf = stored["leaves"][0]
    assert set(leaf) == {"name", "spec", "actor"}
    assert set(leaf["spec"]) == {"shape", "kind", "dtype", "scale", "action_mask", "fields"}
    assert leaf["spec"]["kind"] == "image" and leaf["spec"]["dtype"] == "uint8" and leaf["spec"]["scale"] == 1 / 255
    assert ck.obs_spec_from_json(stored) == obs
    for act in (ActionSpec.discrete(6), ActionSpec.continuous(3, -2.0, 2.0)):
        s = ck.action_spec_to_json(act)
        assert set(s) == {"kind", "n", "dim", "low", "high", "nvec"}
        back = ck.action_spec_from_json(s)
        assert back.kind == act.kind and back.width == act.width
        if act.kind == "continuous":
            assert s["low"] == [-2.0] * 3 and np.array_equal(back.high_array, act.high_array)
    path = _save(tmp_path / "c.npz", obs_spec=obs, action_spec=ActionSpec.discrete(6))
    out = ck.load_checkpoint(path)
    assert out["obs_spec"] == obs and out["action_spec"] == ActionSpec.discrete(6)
    with pytest.raises(ValueError, match="leaves"):
        ck.obs_spec_from_json({"leaves": [leaf, leaf]})
    masked = json.loads(json.dumps(stored))
    masked["leaves"][0]["spec"]["action_mask"] = 4
    with pytest.raises(ValueError, match="action mask"):
        ck.obs_spec_from_json(masked)


def test_write_is_atomic_and_leaves_no_temp_files(tmp_path):
    path = _save(tmp_path / "c.npz")
    _save(tmp_path / "c.npz", agent_state={"w": np.ones(2, np.float32)})
    assert [p.name for p in tmp_path.iterdir()] == ["c.npz"]
    assert np.array_equal(ck.load_checkpoint(path)["agent_state"]["w"], np.ones(2, np.float32))


def _reference_trunk(prefix):
    # The reference exporter's pattern for an actor tower's Linear/conv
    # weights (ttrl/deploy/policies.py:61-66).
    import re
    return re.compile(rf"^{re.escape(prefix)}towers\.(?P<leaf>[^.]+)\.layers\.(?P<index>\d+)\.weight$")


@pytest.mark.parametrize("towers,prefix,ours", [
    ("TOWERS_DQN", "encoder.", ["encoder.layers.0.weight", "encoder.layers.7.weight", "encoder.layers.7.bias",
                                "head.q.weight"]),
    ("TOWERS_SAC", "policy.encoder.", ["policy.encoder.layers.0.weight", "policy.encoder.layers.2.bias",
                                       "policy.head.heads.mean.weight", "critics.0.head.layers.0.weight",
                                       "critics.1.encoder.tower.layers.0.weight",
                                       "targets.1.encoder.tower.layers.0.bias"]),
    ("TOWERS_PPO", "encoders.actor.", ["encoders.actor.layers.0.weight", "encoders.actor.layers.7.weight",
                                       "heads.policy.logits.weight", "heads.value.value.weight",
                                       "memories.actor.cell.weight_ih"]),
])
def test_state_keys_take_the_reference_names_and_come_back(towers, prefix, ours):
    from ttrl_amd.algos import state as st
    table = getattr(st, towers)
    state = {k: i for i, k in enumerate(ours)}
    ref = st.to_reference_keys(state, table, "obs")
    trunk = _reference_trunk(prefix)
    for k in ours:
        if k.startswith(prefix) and k.endswith(".weight"):
            moved = next(r for r, v in ref.items() if v == state[k])
            m = trunk.match(moved)
            assert m and m["leaf"] == "obs" and m["index"] == k.split(".")[-2], moved
    assert "critics.1.encoder.encoder.towers.obs.layers.0.weight" in ref or towers != "TOWERS_SAC"
    assert st.from_reference_keys(ref, table, "obs") == state
    for k in ("head.q.weight", "policy.head.heads.mean.weight", "heads.policy.logits.weight"):
        if k in state:
            assert k in ref  # heads already carry the reference's names


def test_validate_compares_a_reference_config_field_by_field():
    """A reference-written config (a StoredDataclass) is compared on every
    field that maps onto this learner's config; dispatch-only and unmapped
    fields are carried (ttrl/algos/checkpoint.py:107-115 refuses any change)."""
    from ttrl_amd.algos.dqn import DQNConfig
    from ttrl_amd.algos.state import validate
    from ttrl_amd.checkpoint import StoredDataclass

    cfg = DQNConfig(lr=6.25e-5, gamma=0.99, n_step=3, prioritized=True)
    base = {"online": {}, "target": {}, "optimizer": {}, "frame_count": 0, "update_count": 0, "rng_state": {}}

    def state(fields):
        out = dict(base)
        out["config"] = StoredDataclass("ttrl.algos.dqn.config:DQNConfig", fields)
        return out

    kw = dict(algo="DQN", config=cfg, weight_keys=("online", "target"),
              run_keys=("optimizer", "frame_count", "update_count", "rng_state"))
    ok = {"gamma": 0.99, "n_step": 3, "lr": 6.25e-5, "double": True, "step_mode": "traced_fwd_bwd",
          "buffer_capacity": 100000, "priority": {"alpha": 0.6}, "encoder_kwargs": {}}
    assert validate(state(ok), weights_only=False, **kw) is True
    for field, value in (("gamma", 0.9), ("n_step", 1), ("lr", 1e-3), ("double", False),
                         ("target_sync_interval", 1), ("priority", None), ("batch_size", 64)):
        with pytest.raises(ValueError, match="configuration differs") as e:
            validate(state(dict(ok, **{field: value})), weights_only=False, **kw)
        assert field in str(e.value)
        with pytest.raises(ValueError, match="configuration differs"):
            validate(state(dict(ok, **{field: value})), weights_only=True, **kw)
