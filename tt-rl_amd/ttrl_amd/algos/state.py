"""A learner's state tree: a WEIGHTS half (parameters and their lagged
copies) and a RUN half (optimizer moments, counters, the sampling RNG), with
the reference's marker for a weights-only state and its loading rules
(ttrl/algos/checkpoint.py:31-129).

The config is compared as the reference compares it (any difference
refuses the load, ttrl/algos/checkpoint.py:107-115).  A config read from a
reference checkpoint (a `StoredDataclass` of a `ttrl.` class) is compared
field by field wherever a stored field maps onto a field of this learner's
config: the same name, or the reference's `priority` record against this
config's `prioritized` flag.  Fields that only choose how a step is
dispatched (`step_mode`, `act_mode`) are not compared, and stored fields
with no counterpart here are carried.
"""

from __future__ import annotations

import dataclasses
import re

from ttrl_amd.checkpoint import StoredDataclass

__all__ = ["CONFIG_KEY", "WEIGHTS_ONLY_KEY", "TOWERS_DQN", "TOWERS_PPO", "TOWERS_SAC", "assemble",
           "from_reference_keys", "to_reference_keys", "validate"]

WEIGHTS_ONLY_KEY = "weights_only"
CONFIG_KEY = "config"


# Where a network's per-observation towers sit, as (name here, name in the
# reference) templates whose `{field}`s stand for one name segment each.  The
# reference hangs each observation leaf's tower under `<encoder>.towers.<leaf>.`
# (ttrl/nets/multi.py:53-85) and names a critic's concat encoder's tower
# `encoder` (ttrl/nets/fusion.py:60-72); the networks here hold the one
# leaf's tower directly.
TOWERS_DQN = (("encoder", "encoder"),)
TOWERS_SAC = (("policy.encoder", "policy.encoder"), ("{net}.{i}.encoder.tower", "{net}.{i}.encoder.encoder"))
TOWERS_PPO = (("encoders.{role}", "encoders.{role}"),)


def _template(t: str, tail: str) -> re.Pattern:
    parts = re.split(r"\{(\w+)\}", t)
    rx = "".join(re.escape(p) if i % 2 == 0 else f"(?P<{p}>[^.]+)" for i, p in enumerate(parts))
    return re.compile(f"^{rx}{re.escape(tail)}")


def _rename(state: dict, towers, leaf: str, *, to_reference: bool) -> dict:
    out = {}
    for key, value in state.items():
        for here, there in towers:
            src, dst = (here, there) if to_reference else (there, here)
            m = _template(src, "." if to_reference else f".towers.{leaf}.").match(key)
            if m:
                head = dst.format(**m.groupdict())
                key = (f"{head}.towers.{leaf}." if to_reference else f"{head}.") + key[m.end():]
                break
        out[key] = value
    return out


def to_reference_keys(state: dict, towers, leaf: str) -> dict:
    """A network state dict under the reference's parameter names."""
    return _rename(state, towers, leaf, to_reference=True)


def from_reference_keys(state: dict, towers, leaf: str) -> dict:
    """The inverse of `to_reference_keys`; names it does not know pass
    through, so the network's own load names them."""
    return _rename(state, towers, leaf, to_reference=False)


def assemble(config, weights: dict, run: dict, *, weights_only: bool) -> dict:
    """One state dict from its two halves (ttrl/algos/checkpoint.py:31-39)."""
    state = dict(weights)
    state[CONFIG_KEY] = config
    if weights_only:
        state[WEIGHTS_ONLY_KEY] = True
        return state
    state.update(run)
    return state


def _config_diff(saved, current) -> str:
    if not (dataclasses.is_dataclass(saved) and type(saved) is type(current)):
        return f"checkpoint holds {saved!r}; this learner has {current!r}"
    names = [f.name for f in dataclasses.fields(saved) if getattr(saved, f.name) != getattr(current, f.name)]
    was = ", ".join(f"{n}={getattr(saved, n)!r}" for n in names)
    now = ", ".join(f"{n}={getattr(current, n)!r}" for n in names)
    return f"{len(names)} field(s) differ: checkpoint was written with {was}; this learner has {now}"


# Fields that choose how an update is dispatched, not what it computes.
_DISPATCH_ONLY = frozenset({"step_mode", "act_mode", "fused_update"})


def _plain(value):
    """A stored value in comparable form (JSON lists back to tuples)."""
    if isinstance(value, (list, tuple)):
        return tuple(_plain(v) for v in value)
    return value


def _foreign_diff(saved: StoredDataclass, current) -> list:
    """[(field, stored, current)] of mapped fields whose values differ."""
    if not dataclasses.is_dataclass(current):
        return []
    mine = {f.name: getattr(current, f.name) for f in dataclasses.fields(current)}
    out = []
    for name, stored in saved.fields.items():
        if name in _DISPATCH_ONLY:
            continue
        if name == "priority" and "prioritized" in mine:
            if (stored is not None) != bool(mine["prioritized"]):
                out.append(("priority", stored, mine["prioritized"]))
            continue
        if name not in mine or isinstance(stored, (dict, StoredDataclass)):
            continue
        have = mine[name]
        if dataclasses.is_dataclass(have) or isinstance(have, dict):
            continue
        if _plain(stored) != _plain(have):
            out.append((name, stored, have))
    return out


def validate(state: dict, *, algo: str, config, weight_keys: tuple, run_keys: tuple, weights_only: bool) -> bool:
    """Check `state` against what `algo` needs; True when its run half is to
    be loaded (ttrl/algos/checkpoint.py:72-129)."""
    carries_weights_only = bool(state.get(WEIGHTS_ONLY_KEY, False))
    if carries_weights_only and not weights_only:
        raise ValueError(f"{algo}.load_state_dict: this state carries parameters only (written with "
                         f"state_dict(weights_only=True)) and none of {list(run_keys)}; continuing from it would "
                         f"restart the optimizer moments and counters. Pass weights_only=True to load the "
                         f"parameters on purpose.")
    required = tuple(weight_keys) + (CONFIG_KEY,)
    if not (carries_weights_only or weights_only):
        required += tuple(run_keys)
    missing = [key for key in required if key not in state]
    if missing:
        raise ValueError(f"{algo}.load_state_dict: state is missing {missing}.")
    saved = state[CONFIG_KEY]
    if isinstance(saved, StoredDataclass):
        diff = _foreign_diff(saved, config)
        if diff:
            was = ", ".join(f"{n}={a!r}" for n, a, _ in diff)
            now = ", ".join(f"{n}={b!r}" for n, _, b in diff)
            raise ValueError(f"{algo}.load_state_dict: this learner's configuration differs from the state's "
                             f"({saved.path}): {len(diff)} field(s) differ: the state was written with {was}; this "
                             f"learner has {now}. Loading would change the algorithm mid-run.")
    elif saved != config:
        raise ValueError(f"{algo}.load_state_dict: this learner's configuration differs from the state's. "
                         f"{_config_diff(saved, config)}.")
    return not (carries_weights_only or weights_only)
