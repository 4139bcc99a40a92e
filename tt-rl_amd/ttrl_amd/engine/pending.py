"""Work an earlier launch left for the update's optimizer step.

A gradient source (`ttrl_grad_source`) is a parameter gradient left
unreduced: the split-K partial sums of a convolution's weight gradient
(ttrl/engine/conv/backward.py:45-78), or a linear layer's gradients as an
outer product of its input rows and output-gradient rows
(ttrl/engine/layers.py:22-61).  The Adam step over the parameters' arena
forms them as it reads the gradients (`ttrl_adam_step_sources`), so the
update needs no reduction launch per source.  Ordered sums are batch means
(the DQN loss and mean Q, ttrl/algos/dqn/losses.py:120-140) formed by that
step's finishing launch.

Anything that reads a pending gradient before the step (`settle`) or an
update that has no such step (`settle_sums`) writes them with launches of
their own; the values are the same bits either way.
"""

from __future__ import annotations

import ctypes as C

from ttrl_amd import _lib

__all__ = ["PendingGrad", "add_sums", "settle", "settle_sums", "take_sources", "take_sums"]

MAX_SOURCES = 8  # per launch
MAX_SUMS = 4


class PendingGrad:
    """One gradient source and the tensors whose gradients it writes
    (`keep`: device arrays it reads, held until it is formed)."""

    __slots__ = ("source", "tensors", "keep")

    def __init__(self, source: "_lib.GradSource", tensors, keep=()):
        if source.kind == _lib.GRAD_NONE:
            raise ValueError("PendingGrad: nothing pending")
        self.source = source
        self.tensors = [t for t in tensors if t is not None]
        self.keep = tuple(keep)
        for t in self.tensors:
            if t._pending is not None:
                raise RuntimeError("PendingGrad: this gradient is already pending")
            t._pending = self

    def release(self) -> None:
        for t in self.tensors:
            if t._pending is self:
                t._pending = None


def take_sources(tensors) -> "list[PendingGrad]":
    """The distinct pending sources among `tensors`, in order (not released)."""
    out = []
    for t in tensors:
        p = getattr(t, "_pending", None)
        if p is not None and all(p is not q for q in out):
            out.append(p)
    return out


def settle(tensors) -> None:
    """Writes every pending gradient among `tensors` into its buffer."""
    pend = take_sources(tensors)
    if not pend:
        return
    dev = pend[0].tensors[0].device
    for i in range(0, len(pend), MAX_SOURCES):
        chunk = pend[i:i + MAX_SOURCES]
        arr = (_lib.GradSource * len(chunk))(*[p.source for p in chunk])
        dev.call("ttrl_grad_sources_materialize", len(chunk), arr)
        for p in chunk:
            p.release()


def add_sums(dev, sums, keep=()) -> None:
    """Queues ordered sums (`_lib.OrderedSum`) for the device's next step."""
    dev.pending_sums.extend((s, tuple(keep)) for s in sums)


def take_sums(dev) -> list:
    """Removes and returns the queued ordered sums (with their kept arrays)."""
    out = list(dev.pending_sums)
    dev.pending_sums.clear()
    return out


def settle_sums(dev) -> None:
    """Forms the queued ordered sums now, with launches of their own."""
    queued = take_sums(dev)
    for i in range(0, len(queued), MAX_SUMS):
        chunk = [s for s, _ in queued[i:i + MAX_SUMS]]
        arr = (_lib.OrderedSum * len(chunk))(*chunk)
        dev.call("ttrl_ordered_sums", len(chunk), arr)
