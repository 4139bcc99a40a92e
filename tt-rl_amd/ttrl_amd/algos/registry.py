"""Algorithms by name: `ALGOS` and `resolve_and_build`
(ttrl/algos/registry.py:29-51, with the registry verbs of
ttrl/nets/registry.py:71-236).

An entry is a builder `builder(obs_spec, action_spec, device, **kwargs) ->
Agent`, or a "module:attr" string naming one.  String entries are imported
on the first `resolve`, so asking which algorithms exist (`in`, `names`,
`len`, `entry`) imports no learner and opens no device.  A duplicate name and
an unknown name both raise, with the messages the reference gives.
"""

from __future__ import annotations

import importlib
from typing import Callable

__all__ = ["ALGOS", "Registry", "check_agent", "import_target", "resolve_and_build"]


def import_target(target: str) -> Callable:
    """The attribute a "module:attr" entry names, importing its module.  A
    module that does not exist and a module whose own imports fail are
    reported differently: the first is a wrong registration, the second a
    missing dependency (ttrl/nets/registry.py:48-68)."""
    module_name, attr = target.split(":")
    try:
        module = importlib.import_module(module_name)
    except ModuleNotFoundError as exc:
        if exc.name != module_name:
            raise
        raise ModuleNotFoundError(f"the registered target {target!r} names the module {module_name!r}, which does "
                                  f"not exist. Register it as \"<importable module>:{attr}\".") from exc
    if not hasattr(module, attr):
        raise AttributeError(f"the registered target {target!r} names {attr!r} in {module_name!r}, which defines "
                             f"no such name. Register the attribute that is there, or define {attr!r} in "
                             f"{module_name}.")
    return getattr(module, attr)


class Registry:
    """name -> builder, or a "module:attr" target when `allow_targets`."""

    def __init__(self, what: str, *, module: str, allow_targets: bool = False):
        self._what = what
        self._module = module
        self._allow_targets = allow_targets
        self._items: dict[str, Callable | str] = {}

    def register(self, name: str, builder: Callable | str | None = None):
        """Register `builder` under `name`; without a builder, a decorator."""
        if not isinstance(name, str) or not name:
            raise ValueError(f"{self._what} registry: name must be a non-empty string, got {name!r}")
        if name in self._items:
            raise ValueError(
                f"{self._what} registry: {name!r} is already registered to {self._items[name]!r}. Silently "
                f"replacing it would make which {self._what[:-1]} a config names depend on import order. Pick "
                f"another name, or unregister({name!r}) first.")
        if builder is None:
            return self(name)
        if isinstance(builder, str):
            if not self._allow_targets:
                raise TypeError(f"{self._what} registry: builder for {name!r} is not callable. This registry "
                                f"takes callables only.")
            if builder.count(":") != 1:
                raise ValueError(f"{self._what} registry: target {builder!r} for {name!r} must have the form "
                                 f"'module:attr'")
        elif not callable(builder):
            raise ValueError(f"{self._what} registry: builder for {name!r} is not callable")
        self._items[name] = builder
        return builder

    def __call__(self, name: str) -> Callable:
        """Decorator form: `@ALGOS("mine")`."""
        def decorate(builder: Callable) -> Callable:
            self.register(name, builder)
            return builder
        return decorate

    def unregister(self, name: str) -> None:
        if name not in self._items:
            raise KeyError(self._unknown(name))
        del self._items[name]

    def entry(self, name: str) -> Callable | str:
        """The raw entry: a callable, or its "module:attr" target."""
        found = self._items.get(name)
        if found is None:
            raise KeyError(self._unknown(name))
        return found

    def resolve(self, name: str) -> Callable:
        """The builder under `name`, importing a target entry (the one query
        that imports)."""
        found = self.entry(name)
        if isinstance(found, str):
            builder = import_target(found)
            self._items[name] = builder
            return builder
        return found

    def _unknown(self, name: str) -> str:
        if not self._items:
            return (f"the {self._what} registry is empty, which is not a problem with the name {name!r} you "
                    f"passed: nothing registered a builder. Only an explicit "
                    f"{self._module}.{self._what.upper()}.register(name, builder) call can populate it.")
        return (f"unknown {self._what[:-1]} {name!r}; registered names are {self.names()}. Register yours with "
                f"{self._module}.{self._what.upper()}.register(name, builder).")

    def names(self) -> list[str]:
        return sorted(self._items)

    def __contains__(self, name: str) -> bool:
        return name in self._items

    def __len__(self) -> int:
        return len(self._items)


#: `builder(obs_spec, action_spec, device, **kwargs) -> Agent`
ALGOS = Registry("algos", module="ttrl_amd.algos.registry", allow_targets=True)

ALGOS.register("dqn", "ttrl_amd.algos.agents:DQNAgent")
ALGOS.register("ppo", "ttrl_amd.algos.agents:PPOAgent")
ALGOS.register("sac", "ttrl_amd.algos.agents:SACAgent")


def resolve_and_build(name: str, obs_spec, action_spec, device, **kwargs):
    """Resolve an algorithm by name and construct it; unknown names raise
    KeyError (ttrl/algos/registry.py:39-51).  Checks nothing else."""
    return ALGOS.resolve(name)(obs_spec, action_spec, device, **kwargs)


_AGENT_METHODS = ("act", "observe", "should_update", "update", "named_parameters", "parameters", "state_dict",
                  "load_state_dict", "close")


def check_agent(agent) -> None:
    """Raise TypeError unless `agent` carries the whole Agent surface: its
    specs and every method of the protocol (ttrl/algos/checks.py:68-110).
    `Protocol` membership does not check this at construction."""
    from ttrl_amd.spaces import ActionSpec, ObsSpec

    if not isinstance(getattr(agent, "obs_spec", None), ObsSpec):
        raise TypeError(f"{type(agent).__name__} has no obs_spec (an ObsSpec); the trainer reads it to build "
                        f"observations for act()")
    if not isinstance(getattr(agent, "action_spec", None), ActionSpec):
        raise TypeError(f"{type(agent).__name__} has no action_spec (an ActionSpec); the trainer reads it to "
                        f"check the environment's action space")
    missing = [m for m in _AGENT_METHODS if not callable(getattr(agent, m, None))]
    if missing:
        raise TypeError(f"{type(agent).__name__} does not implement the Agent protocol: missing {missing}")
