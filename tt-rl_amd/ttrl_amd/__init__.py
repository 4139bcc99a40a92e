"""ttrl_amd: tt-rl's learner-update path (engine, nets, DQN, SAC and PPO
learners and agents) on AMD MI355X (gfx950) through hand-written HIP
kernels in libttrl_hip.so.

Importing the package loads no library and opens no device; the names
below resolve on first use (ttrl/__init__.py lists the same ones).
"""

from __future__ import annotations

import importlib
from typing import Any

__version__ = "0.1.0"

_LAZY = {
    "ALGOS": "ttrl_amd.algos.registry", "resolve_and_build": "ttrl_amd.algos.registry",
    "check_agent": "ttrl_amd.algos.registry", "Agent": "ttrl_amd.algos.base",
    "Transition": "ttrl_amd.algos.base", "ObsSpec": "ttrl_amd.spaces", "ActionSpec": "ttrl_amd.spaces",
    "acquire": "ttrl_amd.engine.device", "EngineConfig": "ttrl_amd.engine.config",
    "DEFAULT": "ttrl_amd.engine.config",
}

__all__ = sorted(_LAZY)


def __getattr__(name: str) -> Any:
    module = _LAZY.get(name)
    if module is None:
        raise AttributeError(f"module {__name__!r} has no attribute {name!r}")
    return getattr(importlib.import_module(module), name)


def __dir__() -> list[str]:
    return sorted(__all__)
