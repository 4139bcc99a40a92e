"""Checkpoint files: one `.npz` holding every array of a state tree under a
dotted member name, plus a `__meta__` member of UTF-8 JSON that holds the
tree itself with the arrays replaced by markers (ttrl/train/checkpoint/file.py:
87-218, tree.py:65-150, read.py:23-104, specs.py:22-62, atomic.py:24-37).

The container is the reference's, so the files interchange at the level of
the weights: the format token, the level rules (L0 weights snapshot, L1 run
state), the member names (`state.<path>` for the agent state), the markers
(`__array__`, `__bytes__`, `__list__`, `__dataclass__`) and the JSON form of
the observation and action specs are the same, and the learners' state
trees use the reference agents' keys and layouts (`online`/`target`/
`optimizer` for DQN, `nets`/`log_alpha`/`actor_opt`/`critic_opt`/`alpha_opt`
for SAC; OIHW conv weights, (in, out) linear weights, canonical Adam m and v).

Types: a dataclass is stored with its `module:qualname` path.  Reading never
imports a module the file names: a path under this package is rebuilt from
the class already imported here, and any other path (the reference's own
configs, `ttrl.algos.dqn.config:DQNConfig`) comes back as a `StoredDataclass`
record holding the path and the field values, so a reference checkpoint's
weights load without its config class.
"""

from __future__ import annotations

import dataclasses
import importlib
import io
import json
import os
import sys
import uuid
from typing import Any

import numpy as np

from ttrl_amd.spaces import ActionSpec, ObsSpec

__all__ = ["FORMAT", "L0", "L1", "LEVELS", "StoredDataclass", "CheckpointFieldError", "atomic_write", "split", "join",
           "save_checkpoint", "load_checkpoint", "read_meta", "obs_spec_to_json", "obs_spec_from_json",
           "action_spec_to_json", "action_spec_from_json"]

# The reference's on-disk marker (ttrl/train/checkpoint/file.py:100), compared
# for equality only.
FORMAT = "ttrl-checkpoint-9c42ad"
L0 = "L0"
L1 = "L1"
LEVELS = (L0, L1)
_ARRAY_PREFIX = "state"
_META = "__meta__"
# Dataclasses rebuilt on load: only classes of this package.
TYPE_ROOT = "ttrl_amd."


class CheckpointFieldError(ValueError):
    """A stored dataclass field the reading code cannot place."""


@dataclasses.dataclass(frozen=True)
class StoredDataclass:
    """A dataclass from outside this package, as the file stored it."""

    path: str
    fields: dict


# ---------------------------------------------------------------- the tree --

def split(state: Any, prefix: str, arrays: dict) -> Any:
    """The JSON form of `state`; its arrays go into `arrays` under dotted
    names (ttrl/train/checkpoint/tree.py:65-127)."""
    if isinstance(state, np.ndarray):
        arrays[prefix] = state
        return {"__array__": prefix}
    if isinstance(state, (bytes, bytearray)):
        arrays[prefix] = np.frombuffer(bytes(state), dtype=np.uint8)
        return {"__bytes__": prefix}
    if isinstance(state, np.generic):
        return state.item()
    if isinstance(state, StoredDataclass):
        return {"__dataclass__": state.path,
                "fields": {k: split(v, f"{prefix}.{k}", arrays) for k, v in state.fields.items()}}
    if dataclasses.is_dataclass(state) and not isinstance(state, type):
        cls = type(state)
        return {"__dataclass__": f"{cls.__module__}:{cls.__qualname__}",
                "fields": {f.name: split(getattr(state, f.name), f"{prefix}.{f.name}", arrays)
                           for f in dataclasses.fields(state)}}
    if isinstance(state, dict):
        bad = [k for k in state if not isinstance(k, str)]
        if bad:
            raise TypeError(f"checkpoint state at {prefix!r} has non-string keys {bad}: keys become npz member "
                            f"names, so they must be strings.")
        return {k: split(v, f"{prefix}.{k}", arrays) for k, v in state.items()}
    if isinstance(state, (list, tuple)):
        return {"__list__": [split(v, f"{prefix}.{i}", arrays) for i, v in enumerate(state)]}
    if isinstance(state, (str, int, float, bool)) or state is None:
        return state
    raise TypeError(f"checkpoint state at {prefix!r} holds {type(state).__name__}, which has no JSON or array "
                    f"form. A state tree is built from numpy arrays, bytes, numbers, strings, bools, None, lists, "
                    f"dicts and dataclasses.")


def join(node: Any, arrays: dict, *, file: str) -> Any:
    """Rebuild a tree `split` wrote (ttrl/train/checkpoint/tree.py:130-150)."""
    if not isinstance(node, dict):
        return node
    if "__array__" in node or "__bytes__" in node:
        raw = "__bytes__" in node
        key = node["__bytes__"] if raw else node["__array__"]
        if key not in arrays:
            raise ValueError(f"checkpoint at {file!r} references array {key!r}, which the file does not contain: "
                             f"it is truncated or was not written by a ttrl checkpoint writer.")
        return arrays[key].tobytes() if raw else arrays[key]
    if "__list__" in node:
        return [join(v, arrays, file=file) for v in node["__list__"]]
    if "__dataclass__" in node:
        fields = {k: join(v, arrays, file=file) for k, v in node["fields"].items()}
        return _rebuild(node["__dataclass__"], fields, file=file)
    return {k: join(v, arrays, file=file) for k, v in node.items()}


def _rebuild(path: str, fields: dict, *, file: str):
    if not path.startswith(TYPE_ROOT) or path.count(":") != 1:
        return StoredDataclass(path, fields)
    module_name, qualname = path.split(":")
    cls = sys.modules.get(module_name)
    if cls is None:  # a module of this package, never one outside it
        try:
            cls = importlib.import_module(module_name)
        except ImportError:
            cls = None
    for part in qualname.split("."):
        cls = getattr(cls, part, None) if cls is not None else None
    if not (isinstance(cls, type) and dataclasses.is_dataclass(cls)):
        raise CheckpointFieldError(f"checkpoint at {file!r} names the type {path!r}, which is not a dataclass this "
                                   f"build defines.")
    declared = {f.name: f for f in dataclasses.fields(cls)}
    unknown = sorted(k for k in fields if k not in declared)
    if unknown:
        raise CheckpointFieldError(f"checkpoint at {file!r} stores {cls.__name__} field(s) {unknown}, which "
                                   f"{path} does not accept: the field was renamed or removed after the file was "
                                   f"written.")
    missing = sorted(n for n, f in declared.items() if n not in fields and f.init
                     and f.default is dataclasses.MISSING and f.default_factory is dataclasses.MISSING)
    if missing:
        raise CheckpointFieldError(f"checkpoint at {file!r} carries no value for {cls.__name__} field(s) {missing}, "
                                   f"which have no default.")
    kwargs = {k: (tuple(v) if isinstance(v, list) else v) for k, v in fields.items() if declared[k].init}
    return cls(**kwargs)


# ----------------------------------------------------------------- specs --

def obs_spec_to_json(spec: ObsSpec) -> dict:
    """The stored form of a one-leaf observation group
    (`dataclasses.asdict(ObsGroup.of(spec))`, ttrl/train/checkpoint/file.py:176)."""
    return {"leaves": [{"name": spec.name, "actor": True,
                        "spec": {"shape": [int(d) for d in spec.shape], "kind": spec.kind, "dtype": spec.dtype,
                                 "scale": float(spec.scale), "action_mask": 0, "fields": []}}]}


def obs_spec_from_json(stored: dict) -> ObsSpec:
    """Back to an `ObsSpec` (ttrl/train/checkpoint/specs.py:31-45); refuses
    what the learners here do not read: several leaves, masks, fields."""
    leaves = stored.get("leaves") or []
    if len(leaves) != 1:
        raise ValueError(f"checkpoint observation has {len(leaves)} leaves; the learners here read one.")
    leaf = leaves[0]
    s = leaf["spec"]
    if int(s.get("action_mask") or 0) or s.get("fields"):
        raise ValueError("checkpoint observation carries an action mask or named fields, which the learners here "
                         "do not read.")
    return ObsSpec(str(s["kind"]), tuple(int(d) for d in s["shape"]), str(s.get("dtype", "float32")),
                   float(s.get("scale", 1.0)), str(leaf.get("name", "obs")))


def action_spec_to_json(spec: ActionSpec) -> dict:
    """`dataclasses.asdict` of the reference's ActionSpec (kind, n, dim, low,
    high, nvec; ttrl/spaces/action.py)."""
    if spec.kind == "discrete":
        return {"kind": "discrete", "n": int(spec.n), "dim": None, "low": None, "high": None, "nvec": None}
    return {"kind": spec.kind, "n": None, "dim": int(spec.dim), "low": [float(x) for x in spec.low_array],
            "high": [float(x) for x in spec.high_array], "nvec": None}


def action_spec_from_json(stored: dict) -> ActionSpec:
    kind = stored["kind"]
    if kind == "discrete":
        return ActionSpec.discrete(int(stored["n"]))
    if kind == "continuous":
        return ActionSpec.continuous(int(stored["dim"]), tuple(float(x) for x in stored["low"]),
                                     tuple(float(x) for x in stored["high"]))
    raise ValueError(f"checkpoint action kind {kind!r} is not read by the learners here.")


def _json_default(obj: Any) -> Any:
    if isinstance(obj, np.ndarray):
        return obj.tolist()
    if isinstance(obj, np.generic):
        return obj.item()
    raise TypeError(f"object of type {type(obj)!r} is not JSON serializable")


# ------------------------------------------------------------------ files --

def atomic_write(path: str, data: bytes) -> None:
    """Temp file beside the destination, fsync, rename: a reader sees the old
    file or the whole new one (ttrl/train/checkpoint/atomic.py:24-37)."""
    directory = os.path.dirname(os.path.abspath(path)) or "."
    os.makedirs(directory, exist_ok=True)
    tmp = os.path.join(directory, f".{os.path.basename(path)}.tmp-{uuid.uuid4().hex}")
    fd = os.open(tmp, os.O_WRONLY | os.O_CREAT | os.O_EXCL, 0o644)
    try:
        with os.fdopen(fd, "wb") as fh:
            fh.write(data)
            fh.flush()
            os.fsync(fh.fileno())
        os.replace(tmp, path)
    except BaseException:
        try:
            os.remove(tmp)
        except OSError:
            pass
        raise


def save_checkpoint(path: str, *, agent_state: dict, obs_spec: ObsSpec, action_spec: ActionSpec, level: str = L1,
                    frame: int = 0, config=None, env_policy_state: list | None = None,
                    env_reward_state: list | None = None, replay_state: dict | None = None,
                    cadence_state: dict | None = None, extra: dict | None = None) -> None:
    """Write a checkpoint atomically (ttrl/train/checkpoint/file.py:112-218):
    the same level rules, members and meta."""
    if level not in LEVELS:
        raise ValueError(f"level must be one of {LEVELS}, got {level!r}.")
    if level == L0:
        for name, value in (("replay_state", replay_state), ("env_reward_state", env_reward_state),
                            ("cadence_state", cadence_state)):
            if value:
                raise ValueError(f"an L0 checkpoint is a weights snapshot and carries no run state, but {name} "
                                 f"was given; write it to an L1 file.")
    if level == L1 and config is None:
        raise ValueError("an L1 checkpoint carries the run config; pass config=, or write level='L0' for a "
                         "weights snapshot.")
    arrays: dict = {}
    meta: dict = {
        "format": FORMAT,
        "level": level,
        "obs_spec": obs_spec_to_json(obs_spec),
        "action_spec": action_spec_to_json(action_spec),
        "agent_state": split(agent_state, _ARRAY_PREFIX, arrays),
        "env_policy_state": None if env_policy_state is None else split(env_policy_state, "env_policy_state", arrays),
        "extra": extra or {},
    }
    if level == L1:
        meta["frame"] = int(frame)
        meta["config"] = split(config, "config", arrays)
        meta["env_reward_state"] = (None if env_reward_state is None
                                    else split(env_reward_state, "env_reward_state", arrays))
        meta["replay_state"] = None if replay_state is None else split(replay_state, "replay_state", arrays)
        meta["cadence_state"] = None if cadence_state is None else split(cadence_state, "cadence_state", arrays)
    payload = dict(arrays)
    payload[_META] = np.frombuffer(json.dumps(meta, default=_json_default).encode("utf-8"), dtype=np.uint8)
    buf = io.BytesIO()
    np.savez(buf, **payload)
    atomic_write(path, buf.getvalue())


def read_meta(path: str) -> tuple[dict, dict]:
    """The raw arrays and meta of a checkpoint, the format marker checked
    (ttrl/train/checkpoint/read.py:23-44).  Loads nothing executable."""
    try:
        with np.load(path, allow_pickle=False) as npz:
            meta = json.loads(npz[_META].tobytes().decode("utf-8"))
            arrays = {k: npz[k] for k in npz.files if k != _META}
    except Exception as exc:
        raise ValueError(f"{path!r} is not a readable ttrl checkpoint: {type(exc).__name__}: {exc}") from exc
    if meta.get("format") != FORMAT:
        raise ValueError(f"{path!r} does not carry the checkpoint format marker {FORMAT!r} (it carries "
                         f"{meta.get('format')!r}).")
    return arrays, meta


def load_checkpoint(path: str) -> dict:
    """`level`, `obs_spec`, `action_spec`, `agent_state`, `env_policy_state`,
    `extra`, and for L1 `frame`, `config`, `env_reward_state`,
    `replay_state`, `cadence_state` (ttrl/train/checkpoint/read.py:47-104)."""
    arrays, meta = read_meta(path)

    def opt(key):
        return join(meta[key], arrays, file=path) if meta.get(key) is not None else None

    out = {"level": meta["level"], "obs_spec": obs_spec_from_json(meta["obs_spec"]),
           "action_spec": action_spec_from_json(meta["action_spec"]),
           "agent_state": join(meta["agent_state"], arrays, file=path),
           "env_policy_state": opt("env_policy_state"), "extra": meta.get("extra") or {}}
    if meta["level"] == L1:
        out["frame"] = int(meta["frame"])
        out["config"] = join(meta["config"], arrays, file=path)
        for key in ("env_reward_state", "replay_state", "cadence_state"):
            out[key] = opt(key)
    return out
