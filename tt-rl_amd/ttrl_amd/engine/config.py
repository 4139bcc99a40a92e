"""EngineConfig: the engine settings a caller states explicitly
(ttrl/engine/config.py:10-24, same fields and defaults).

`trace_blocking` means here what it means in the reference: whether a
replay of a captured step waits for the device before returning
(ttrl/engine/step/core.py:87-91, :135-141).  The two sizes are allocator
reservations a Tenstorrent chip needs at open time; a HIP context needs
neither (graphs and the conv workspace are allocated on demand), so they
are accepted at their defaults and a different value is refused rather
than silently ignored.
"""

from __future__ import annotations

from dataclasses import dataclass, fields

__all__ = ["EngineConfig", "DEFAULT", "check_engine_config"]


@dataclass(frozen=True)
class EngineConfig:
    # Whether a replay waits for the device before returning.
    trace_blocking: bool = False
    # Tenstorrent L1 "small" pool reservation; no counterpart on a GPU.
    l1_small_size: int = 32768
    # Tenstorrent trace-region reservation; no counterpart on a GPU.
    trace_region_size: int = 32 * 1024 * 1024


DEFAULT = EngineConfig()

_NO_COUNTERPART = ("l1_small_size", "trace_region_size")


def check_engine_config(cfg, who: str) -> EngineConfig:
    """`cfg` as an EngineConfig (None means DEFAULT); a field without a
    meaning on this device set away from its default raises ValueError."""
    if cfg is None:
        return DEFAULT
    if not isinstance(cfg, EngineConfig):
        names = [f.name for f in fields(EngineConfig)]
        raise ValueError(f"{who}: cfg must be an EngineConfig (fields {names}), got {type(cfg).__name__}")
    for name in _NO_COUNTERPART:
        value, default = getattr(cfg, name), getattr(DEFAULT, name)
        if value != default:
            raise ValueError(
                f"{who}: EngineConfig.{name}={value!r} sizes a Tenstorrent allocator region that a HIP device "
                f"does not have (graphs and workspaces are allocated as needed); leave it at its default "
                f"{default!r}.")
    return cfg
