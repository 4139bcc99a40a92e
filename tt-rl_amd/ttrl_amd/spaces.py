"""Observation and action specs, the subset the learner path reads
(ttrl/spaces/obs.py:83-248, ttrl/spaces/action.py:16-150): an image leaf is
uint8 (C, H, W) with scale 1/255, a vector leaf float32 (n,) with scale 1;
actions are discrete(n) or continuous(dim, low, high)."""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

__all__ = ["ObsSpec", "ActionSpec"]


@dataclass(frozen=True)
class ObsSpec:
    kind: str
    shape: tuple
    dtype: str = "float32"
    scale: float = 1.0
    name: str = "obs"

    @staticmethod
    def image(shape=(4, 84, 84), name: str = "obs") -> "ObsSpec":
        if len(tuple(shape)) != 3:
            raise ValueError(f"ObsSpec.image: shape must be (C, H, W), got {shape}")
        return ObsSpec("image", tuple(int(d) for d in shape), "uint8", 1.0 / 255.0, name)

    @staticmethod
    def vector(size: int, name: str = "obs", scale: float = 1.0) -> "ObsSpec":
        return ObsSpec("vector", (int(size),), "float32", float(scale), name)

    @property
    def size(self) -> int:
        return int(np.prod(self.shape))


@dataclass(frozen=True)
class ActionSpec:
    kind: str
    n: int = 0
    dim: int = 0
    low: float | tuple = -1.0
    high: float | tuple = 1.0

    @staticmethod
    def discrete(n: int) -> "ActionSpec":
        if n < 1:
            raise ValueError(f"ActionSpec.discrete: n must be >= 1, got {n}")
        return ActionSpec("discrete", n=int(n))

    @staticmethod
    def continuous(dim: int, low=-1.0, high=1.0) -> "ActionSpec":
        if dim < 1:
            raise ValueError(f"ActionSpec.continuous: dim must be >= 1, got {dim}")
        return ActionSpec("continuous", dim=int(dim), low=low, high=high)

    @property
    def width(self) -> int:
        return self.n if self.kind == "discrete" else self.dim

    @property
    def low_array(self) -> np.ndarray:
        return np.broadcast_to(np.asarray(self.low, np.float32), (self.dim,)).astype(np.float32)

    @property
    def high_array(self) -> np.ndarray:
        return np.broadcast_to(np.asarray(self.high, np.float32), (self.dim,)).astype(np.float32)
