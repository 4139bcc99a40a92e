"""Conv tower specs (ttrl/nets/towers.py:40): the Nature CNN (Mnih et al.
2015) as (out_channels, kernel, stride, padding) stages."""

from __future__ import annotations

from typing import NamedTuple


class ConvStage(NamedTuple):
    out_channels: int
    kernel: int
    stride: int
    padding: int = 0


NATURE_CNN = (ConvStage(32, 8, 4), ConvStage(64, 4, 2), ConvStage(64, 3, 1))
