"""Learners and agents on the MI355X path: DQN (double, n-step, prioritized
weights), SAC (twin critics, learned temperature) and PPO (clipped,
shared trunk), and the registry that resolves one by name
(ttrl/algos/__init__.py:1-60).

Lazy: importing this package imports no learner and opens no device;
`ALGOS` answers which algorithms exist without importing them.
"""

from __future__ import annotations

import importlib
from typing import Any

from ttrl_amd.algos.registry import ALGOS, check_agent, resolve_and_build

_LAZY = {
    "Agent": "base", "AutoresetTracker": "base", "Transition": "base",
    "DQN": "agents", "DQNAgent": "agents", "DQNConfig": "dqn", "DQNLearner": "dqn",
    "PPO": "agents", "PPOAgent": "agents", "PPOConfig": "ppo", "PPOLearner": "ppo",
    "SAC": "agents", "SACAgent": "agents", "SACConfig": "sac", "SACLearner": "sac",
}

#: the reference's class names for the agents
_ALIASES = {"DQN": "DQNAgent", "PPO": "PPOAgent", "SAC": "SACAgent"}

__all__ = ["ALGOS", "check_agent", "resolve_and_build", *sorted(_LAZY)]


def __getattr__(name: str) -> Any:
    module = _LAZY.get(name)
    if module is None:
        raise AttributeError(f"module {__name__!r} has no attribute {name!r}")
    return getattr(importlib.import_module(f"ttrl_amd.algos.{module}"), _ALIASES.get(name, name))


def __dir__() -> list[str]:
    return sorted(__all__)
