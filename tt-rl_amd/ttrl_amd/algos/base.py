"""What a train loop may do to an agent (ttrl/algos/base.py:40-253): the
`Transition` one vector-env step hands over, the `Agent` protocol, and the
autoreset bookkeeping that keeps padding steps out of replay.

Observations are lane-major arrays of this package's single observation
leaf; a mapping {leaf name: array} (the reference's Observation over one
leaf) is accepted wherever an observation is.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Iterator, Mapping, Protocol, runtime_checkable

import numpy as np

__all__ = ["Agent", "AutoresetTracker", "Transition", "leaf_array"]


def leaf_array(obs, name: str | None = None) -> np.ndarray:
    """The lane-major array of an observation given as an array or a
    one-leaf mapping (named `name` when given)."""
    if isinstance(obs, Mapping):
        if name is not None and name in obs:
            return np.asarray(obs[name])
        if len(obs) != 1:
            raise ValueError(f"expected an observation of one leaf, got leaves {sorted(obs)}")
        return np.asarray(next(iter(obs.values())))
    return np.asarray(obs)


@dataclass
class Transition:
    """One vector-env step, every field lane-major (ttrl/algos/base.py:40-96).

    Under the NEXT_STEP autoreset contract a lane that ends its episode
    returns that episode's final observation as its `next_obs`; the lane's
    following step is the autoreset padding step, dropped by
    `AutoresetTracker`."""

    obs: Any
    action: np.ndarray
    reward: np.ndarray
    terminated: np.ndarray
    truncated: np.ndarray
    next_obs: Any

    def __post_init__(self) -> None:
        lanes = leaf_array(self.obs).shape[0]
        for field in ("action", "reward", "terminated", "truncated"):
            n = np.asarray(getattr(self, field)).shape[0]
            if n != lanes:
                raise ValueError(f"Transition: {field} covers {n} lanes but obs covers {lanes}; every field is "
                                 f"lane-major over one vector env")
        if leaf_array(self.next_obs).shape != leaf_array(self.obs).shape:
            raise ValueError(f"Transition: next_obs has shape {leaf_array(self.next_obs).shape} and obs "
                             f"{leaf_array(self.obs).shape}; pass the successor of every lane, final observations "
                             f"included")

    @property
    def n_envs(self) -> int:
        return int(leaf_array(self.obs).shape[0])

    @property
    def done(self) -> np.ndarray:
        return np.asarray(self.terminated, bool) | np.asarray(self.truncated, bool)


@runtime_checkable
class Agent(Protocol):
    """The agent contract of ttrl/algos/base.py:118-187."""

    def act(self, obs, *, deterministic: bool = False, episode_starts=None) -> np.ndarray: ...

    def named_parameters(self) -> Iterator[tuple[str, Any]]: ...

    def parameters(self) -> Iterator[Any]: ...

    def observe(self, transition: Transition) -> None: ...

    def update(self) -> dict: ...

    def should_update(self, frame: int) -> bool: ...

    def state_dict(self, *, weights_only: bool = False) -> dict: ...

    def load_state_dict(self, state: dict, *, weights_only: bool = False) -> None: ...

    def close(self) -> None: ...


class AutoresetTracker:
    """Which lanes of a step are real transitions (ttrl/algos/base.py:190-253).

    The step after a lane reports done is that lane's autoreset step (its
    action ignored, its reward made up), so it is not a transition; which
    lanes those are follows from the previous step's done flags."""

    def __init__(self, n_envs: int):
        if int(n_envs) < 1:
            raise ValueError(f"AutoresetTracker: n_envs must be >= 1, got {n_envs}")
        self.n_envs = int(n_envs)
        self._after_done = np.zeros(self.n_envs, bool)

    @property
    def pending(self) -> np.ndarray:
        return self._after_done.copy()

    def valid(self, transition: Transition) -> np.ndarray:
        if transition.n_envs != self.n_envs:
            raise ValueError(f"AutoresetTracker: a step of {transition.n_envs} lanes, built for {self.n_envs}")
        done = transition.done
        clash = np.flatnonzero(self._after_done & done)
        if clash.size:
            raise ValueError(f"lanes {clash.tolist()} report done on their autoreset step; under the NEXT_STEP "
                             f"contract the step after an episode's end reports done False")
        real = ~self._after_done
        self._after_done = done.copy()
        return real

    def state_dict(self) -> dict:
        return {"pending": self._after_done.copy()}

    def load_state_dict(self, state: dict) -> None:
        """Checks the stored lane count, then starts with no lane pending: a
        restored run resets its environments before the next step."""
        pending = np.asarray(state["pending"], bool)
        if pending.shape != (self.n_envs,):
            raise ValueError(f"AutoresetTracker: stored pending flags have shape {pending.shape}, expected "
                             f"{(self.n_envs,)}")
        self._after_done = np.zeros(self.n_envs, bool)
