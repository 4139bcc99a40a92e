"""Checkpoint in, deployable policy artifact out, and an artifact run on the
MI355X (ttrl/deploy/export.py:77-254, read.py:23-75, policies.py:40-115,
towers.py:17-73).

`export_policy` writes the reference's artifact: the actor's conv stages
(`conv.<i>.weight` in OIHW with the observation scale folded into the first,
`conv.<i>.bias`), its Linear trunk (`trunk.<i>.weight` (in, out), a vector
policy's observation scale folded into the first), the head, the action
bounds for a bounded map, and a `__meta__` JSON member with the format
marker, the action map and the conv geometry.  The actor is found by name in
the agent state, as the reference's source table names it, so the file is
what the reference's `load_policy` reads.

`load_policy(path, device)` builds the artifact's network on the GPU, with
the folded scale (observation scale 1), and returns a `DeployedPolicy` whose
call runs the fused acting step: the first-index argmax of the head for an
`argmax` map, tanh of the mean mapped onto the bounds for `tanh_bounds`.
"""

from __future__ import annotations

import io
import json
import re
from dataclasses import dataclass, field

import numpy as np

from ttrl_amd.checkpoint import StoredDataclass, atomic_write, load_checkpoint
from ttrl_amd.nets.towers import NATURE_CNN
from ttrl_amd.spaces import ActionSpec, ObsSpec

__all__ = ["ARTIFACT_FORMAT", "ACTION_MAPS", "META_KEY", "DeployedPolicy", "export_policy", "load_policy",
           "read_artifact"]

# The reference's artifact marker (ttrl/deploy/read.py:29), compared for
# equality only, and its JSON member.
ARTIFACT_FORMAT = "ttrl-policy-9c2e57"
META_KEY = "__meta__"
# Action map -> whether it needs the action bounds (ttrl/deploy/artifact.py:63-67).
ACTION_MAPS = {"tanh_bounds": True, "clip_bounds": True, "argmax": False}
# The image towers whose strides an export can read, by encoder name.
TOWERS = {"nature_cnn": NATURE_CNN}


@dataclass(frozen=True)
class _Source:
    """Where one algorithm's actor is (ttrl/deploy/policies.py:40-98)."""

    algo: str
    config: str  # the config class's name
    state_key: str
    trunk: str  # prefix of the actor tower's parameters
    heads: dict = field(compare=False)
    maps: dict = field(compare=False)
    memory: str | None = None


SOURCES = (
    _Source("sac", "SACConfig", "nets", "policy.encoder.", {"continuous": "policy.head.heads.mean.weight"},
            {"continuous": "tanh_bounds"}),
    _Source("ppo", "PPOConfig", "net", "encoders.actor.",
            {"continuous": "heads.policy.heads.mean.weight", "discrete": "heads.policy.logits.weight"},
            {"continuous": "clip_bounds", "discrete": "argmax"}, memory="memories."),
    _Source("dqn", "DQNConfig", "online", "encoder.", {"discrete": "head.q.weight"}, {"discrete": "argmax"}),
)


def _refuse(ok: bool, path: str, complaint: str) -> None:
    if not ok:
        raise ValueError(f"cannot export a deployable policy: {path!r} {complaint}.")


def _config_name(config) -> str:
    if isinstance(config, StoredDataclass):
        return config.path.rsplit(":", 1)[-1].rsplit(".", 1)[-1]
    return type(config).__name__


def _config_field(config, name: str, default):
    if isinstance(config, StoredDataclass):
        return config.fields.get(name, default)
    return getattr(config, name, default)


def _source_for(config, path: str) -> _Source:
    name = _config_name(config)
    for source in SOURCES:
        if source.config == name:
            return source
    raise ValueError(f"cannot export a deployable policy: {path!r} was trained with {name}, and this exporter "
                     f"knows {', '.join(s.config for s in SOURCES)}.")


def _actor(nets: dict, source: _Source, kind: str, path: str):
    """The actor's layers by name: its tower in order, then its head
    (ttrl/deploy/export.py:199-241)."""
    memory = sorted(k for k in nets if source.memory and k.startswith(source.memory))
    _refuse(not memory, path, f"holds a recurrent {source.algo} policy (memory parameters {memory[:2]}...), and "
            f"the artifact is a feedforward map with no carried state")
    head_key = source.heads[kind]
    _refuse(head_key in nets, path, f"holds no parameter named {head_key!r}, where {source.algo}'s {kind} head lives")
    pattern = re.compile(rf"^{re.escape(source.trunk)}towers\.(?P<leaf>[^.]+)\.layers\.(?P<index>\d+)\.weight$")
    layers = {}
    for key in nets:
        m = pattern.match(key)
        if m:
            layers[int(m["index"])] = key
    _refuse(bool(layers), path, f"holds no actor tower matching {pattern.pattern!r}")

    def pair(weight_key):
        return np.asarray(nets[weight_key], np.float32), np.asarray(nets[weight_key[:-len("weight")] + "bias"],
                                                                    np.float32)

    return [pair(layers[i]) for i in sorted(layers)], pair(head_key)


def _split_tower(trunk: list, obs_spec: ObsSpec, config, path: str):
    """(conv stages with the scale folded into the first, their geometry, the
    Linear trunk) (ttrl/deploy/towers.py:17-73)."""
    convs = [layer for layer in trunk if layer[0].ndim == 4]
    linears = trunk[len(convs):]
    _refuse(all(layer[0].ndim == 2 for layer in linears), path,
            "has an actor tower whose convolutions do not all precede its Linear layers")
    if obs_spec.kind != "image":
        _refuse(not convs, path, f"has convolution weights in an actor reading {obs_spec.kind} observations")
        return [], [], linears
    encoder = _config_field(config, "encoder", "auto")
    name = "nature_cnn" if encoder == "auto" else encoder
    _refuse(name in TOWERS, path, f"was trained with the image encoder {name!r}; the exporter reads the strides of "
            f"{sorted(TOWERS)}")
    tower = TOWERS[name]
    _refuse(len(convs) == len(tower), path, f"has {len(convs)} conv stages where the {name!r} tower has {len(tower)}")
    channels, height, width = obs_spec.shape
    stages, geometry = [], []
    for index, ((weight, bias), stage) in enumerate(zip(convs, tower)):
        expected = (stage.out_channels, channels, stage.kernel, stage.kernel)
        _refuse(weight.shape == expected, path,
                f"has conv stage {index} weight of shape {weight.shape} where the {name!r} tower builds {expected}")
        height = (height + 2 * stage.padding - stage.kernel) // stage.stride + 1
        width = (width + 2 * stage.padding - stage.kernel) // stage.stride + 1
        channels = stage.out_channels
        scale = np.float32(obs_spec.scale if index == 0 else 1.0)
        stages.append((weight * scale, bias.reshape(-1)))
        geometry.append({"stride": stage.stride, "padding": stage.padding})
    features = channels * height * width
    _refuse(bool(linears) and linears[0][0].shape[0] == features, path,
            f"has a conv tower ending in {channels}x{height}x{width} = {features} features and no Linear reading them")
    return stages, geometry, linears


def export_policy(checkpoint_path: str, out_path: str) -> str:
    """Write the actor of `checkpoint_path` to `out_path` as the reference's
    policy artifact; returns `out_path` (ttrl/deploy/export.py:77-180)."""
    path = checkpoint_path
    loaded = load_checkpoint(path)
    obs_spec, action_spec = loaded["obs_spec"], loaded["action_spec"]
    state = loaded["agent_state"]
    source = _source_for(state.get("config"), path)
    kind = action_spec.kind
    _refuse(kind in source.maps, path, f"was trained with {source.algo} on a {kind} action spec, which has no "
            f"action map here")
    action_map = source.maps[kind]
    nets = state.get(source.state_key)
    _refuse(isinstance(nets, dict), path, f"carries no {source.state_key!r} member of parameters")
    trunk, head = _actor(nets, source, kind, path)
    stages, geometry, trunk = _split_tower(trunk, obs_spec, state.get("config"), path)
    _refuse(bool(stages) or trunk[0][0].shape[0] == obs_spec.size, path,
            f"has an actor trunk reading {trunk[0][0].shape[0]} inputs for an observation of {obs_spec.size}")
    width = head[0].shape[1]
    _refuse(width == action_spec.width, path, f"has a policy head emitting {width} numbers for an action spec of "
            f"width {action_spec.width}")
    policy_state = loaded["env_policy_state"]
    _refuse(not policy_state, path, "carries an observation transform state, which this exporter does not write")
    if not stages:  # a vector trunk's first Linear takes the observation scale
        trunk[0] = (trunk[0][0] * np.float32(obs_spec.scale), trunk[0][1])
    arrays = {}
    for index, (weight, bias) in enumerate(stages):
        arrays[f"conv.{index}.weight"] = weight
        arrays[f"conv.{index}.bias"] = bias
    for index, (weight, bias) in enumerate(trunk):
        arrays[f"trunk.{index}.weight"] = weight
        arrays[f"trunk.{index}.bias"] = bias.reshape(-1)
    arrays["head.weight"], arrays["head.bias"] = head[0], head[1].reshape(-1)
    if ACTION_MAPS[action_map]:
        arrays["action_low"] = action_spec.low_array.astype(np.float32)
        arrays["action_high"] = action_spec.high_array.astype(np.float32)
    meta = {
        "artifact_format": ARTIFACT_FORMAT,
        "algo": source.algo,
        "action_kind": kind,
        "action_map": action_map,
        "obs_dim": None if stages else int(obs_spec.size),
        "obs_shape": [int(d) for d in obs_spec.shape],
        "conv": geometry,
        "privileged_fields": [],
        "action_dim": int(action_spec.dim) if kind == "continuous" else None,
        "n_actions": int(action_spec.n) if kind == "discrete" else None,
        "action_mask": 0,
        "trunk_layers": len(trunk),
        "normalizer": None,
        "source_checkpoint": checkpoint_path,
    }
    payload = dict(arrays)
    payload[META_KEY] = np.frombuffer(json.dumps(meta).encode("utf-8"), dtype=np.uint8)
    buf = io.BytesIO()
    np.savez(buf, **payload)
    atomic_write(out_path, buf.getvalue())
    return out_path


def read_artifact(path: str) -> tuple[dict, dict]:
    """An artifact's (meta, arrays), its marker checked
    (ttrl/deploy/read.py:38-70).  Loads nothing executable."""
    with np.load(path, allow_pickle=False) as npz:
        if META_KEY not in npz.files:
            raise ValueError(f"{path!r} has no {META_KEY!r} member, so it is not a policy artifact.")
        meta = json.loads(npz[META_KEY].tobytes().decode("utf-8"))
        arrays = {k: npz[k] for k in npz.files if k != META_KEY}
    if "artifact_format" not in meta and "format" in meta:
        raise ValueError(f"{path!r} is a ttrl CHECKPOINT (format marker {meta['format']!r}) rather than a policy "
                         f"artifact; turn it into one with export_policy(checkpoint_path, artifact_path).")
    if meta.get("artifact_format") != ARTIFACT_FORMAT:
        raise ValueError(f"{path!r} does not carry the policy artifact marker {ARTIFACT_FORMAT!r} (it carries "
                         f"{meta.get('artifact_format')!r}).")
    return meta, arrays


class DeployedPolicy:
    """An artifact's deterministic action, computed by the acting kernels.

    `policy(obs)` takes one observation of `obs_shape` or a batch of up to
    `lanes`; a discrete policy returns int64 action indices (a scalar for one
    observation), a continuous one actions in the environment's units."""

    def __init__(self, meta: dict, arrays: dict, device, *, lanes: int = 1, mode: str = "graph"):
        from ttrl_amd.algos.gaussian import ActionScale
        from ttrl_amd.nets.acting import ActingNet, GreedyDecision, SquashedDecision
        from ttrl_amd.nets.build import build_encoder, build_q_net
        from ttrl_amd.nets.heads import GaussianHead
        from ttrl_amd.nets.models import EncoderHead

        self.algo, self.action_map = meta["algo"], meta["action_map"]
        if self.action_map not in ("argmax", "tanh_bounds"):
            raise ValueError(f"DeployedPolicy runs the 'argmax' and 'tanh_bounds' maps on the device; this artifact's "
                             f"map is {self.action_map!r}")
        if int(meta.get("action_mask") or 0) or meta.get("normalizer") is not None:
            raise ValueError("DeployedPolicy: artifacts with a legal-action mask or an observation normaliser are "
                             "not run here")
        self.obs_shape = tuple(int(d) for d in meta["obs_shape"])
        n_conv = len(meta["conv"])
        if n_conv:
            geometry = [(g["stride"], g["padding"]) for g in meta["conv"]]
            if geometry != [(s.stride, s.padding) for s in NATURE_CNN]:
                raise ValueError(f"DeployedPolicy: conv geometry {geometry} is not the Nature CNN's")
            obs_spec = ObsSpec("image", self.obs_shape, "uint8", 1.0)  # the scale is folded into conv.0
        else:
            obs_spec = ObsSpec.vector(int(meta["obs_dim"]))
        self.lanes = int(lanes)
        layers = [(arrays[f"conv.{i}.weight"], arrays[f"conv.{i}.bias"]) for i in range(n_conv)]
        layers += [(arrays[f"trunk.{i}.weight"], arrays[f"trunk.{i}.bias"]) for i in range(int(meta["trunk_layers"]))]
        head = (arrays["head.weight"], arrays["head.bias"])
        hidden = tuple(int(w.shape[1]) for w, _ in layers[n_conv:])
        kwargs = {"hidden": hidden[0]} if n_conv else {"hidden": hidden}
        if self.action_map == "argmax":
            self.n_actions = int(meta["n_actions"])
            net = build_q_net(obs_spec, ActionSpec.discrete(self.n_actions), device, batch=self.lanes, **kwargs)
            decision = GreedyDecision()
            head_keys = ("head.q.weight", "head.q.bias")
        else:
            self.action_dim = int(meta["action_dim"])
            spec = ActionSpec.continuous(self.action_dim, tuple(arrays["action_low"].tolist()),
                                         tuple(arrays["action_high"].tolist()))
            encoder = build_encoder(obs_spec, device, batch=self.lanes, **kwargs)
            net = EncoderHead(encoder, GaussianHead(encoder.out_features, self.action_dim, device))
            decision = SquashedDecision(ActionScale(spec, device))
            head_keys = ("head.heads.mean.weight", "head.heads.mean.bias")
        state = net.state_dict()
        index = sorted({int(m[1]) for k in state if (m := re.match(r"^encoder\.layers\.(\d+)\.weight$", k))})
        if len(index) != len(layers):
            raise ValueError(f"DeployedPolicy: the artifact has {len(layers)} layers and the network {len(index)}")
        new = {k: np.zeros_like(v) for k, v in state.items()}
        for i, (w, b) in zip(index, layers):
            wk, bk = f"encoder.layers.{i}.weight", f"encoder.layers.{i}.bias"
            if tuple(np.shape(w)) != tuple(state[wk].shape):
                raise ValueError(f"DeployedPolicy: layer {i} weight {np.shape(w)} does not fit {state[wk].shape}")
            new[wk], new[bk] = np.asarray(w, np.float32), np.asarray(b, np.float32).reshape(state[bk].shape)
        new[head_keys[0]] = np.asarray(head[0], np.float32)
        new[head_keys[1]] = np.asarray(head[1], np.float32).reshape(state[head_keys[1]].shape)
        net.load_state_dict(new)
        self._net = net
        self._acting = ActingNet(net, obs_spec, device, width=self.lanes, lanes=self.lanes, decision=decision,
                                 mode=mode)

    def __call__(self, obs) -> np.ndarray:
        arr = np.asarray(obs)
        single = arr.ndim == len(self.obs_shape)
        rows = arr.reshape((-1,) + self.obs_shape)
        out = self._acting.decide(rows, deterministic=True)
        if self.action_map == "argmax":
            act = np.asarray(out["actions"]).astype(np.int64).reshape(-1)
        else:
            act = np.asarray(out["action"], np.float32).reshape(-1, self.action_dim)
        return act[0] if single else act

    def close(self) -> None:
        self._acting.close()


def load_policy(path: str, device, *, lanes: int = 1, mode: str = "graph") -> DeployedPolicy:
    """Read an artifact `export_policy` (or the reference's) wrote and build
    it on the GPU for up to `lanes` observations per call."""
    return DeployedPolicy(*read_artifact(path), device, lanes=lanes, mode=mode)
