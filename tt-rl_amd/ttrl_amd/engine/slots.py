"""Input slots: an update captured once per bound input block, so a batch
is read where it was written.

The reference's step has one bound block that every batch is written into
before the run (ttrl/engine/step/inputs.py:16-102, step/core.py:21-160).
With input slots the step holds n blocks of one layout and one graph per
block: the caller writes a batch into slot k's block (a replay draw
assembling it in place, a device copy, a host upload) and launches slot k,
which reads it there.  A loop that draws several batches at once gives
each its own slot and runs the updates back to back, with no copy of a
batch into a fixed block between them.

Everything runs on the context's one stream, so a write into slot k queued
after the launch of an update that reads slot k waits for that update.
"""

from __future__ import annotations

from ttrl_amd.engine.autograd import Tensor
from ttrl_amd.engine.tensor import DeviceArray, _Block

__all__ = ["InputSlots", "MAX_SLOTS", "check_slot_count", "metric_ptrs", "twin_inputs"]

MAX_SLOTS = 64


def metric_ptrs(metrics: dict | None) -> dict:
    """{name: device address} of a step's tensor metrics: every slot's graph
    must write its metrics to the same buffers."""
    return {k: v.data.ptr for k, v in (metrics or {}).items() if isinstance(v, Tensor)}


def twin_inputs(device, inputs: dict) -> dict:
    """A fresh block of `inputs["_block"]`'s size with an input view at the
    same offset, shape and dtype for every input of that block; inputs
    outside the block are shared."""
    block = inputs["_block"]
    fresh = _Block(device, block.block.nbytes)
    whole = DeviceArray(device, block.shape, block.dtype, block=fresh, offset=block.offset)
    out = {"_block": whole}
    for name, t in inputs.items():
        if name == "_block":
            continue
        d = getattr(t, "data", None)
        if isinstance(d, DeviceArray) and d.same_storage(block):
            out[name] = Tensor(DeviceArray(device, d.shape, d.dtype, block=fresh, offset=d.offset))
        else:
            out[name] = t
    return out


def check_slot_count(who: str, n: int) -> None:
    if not 2 <= n <= MAX_SLOTS:
        raise ValueError(f"{who}: {n} input slots; between 2 and {MAX_SLOTS} are supported")


class InputSlots:
    """The slots of one captured update: graphs[k] reads blocks[k]."""

    def __init__(self, device, blocks: list):
        check_slot_count("InputSlots", len(blocks))
        if any(b.nbytes != blocks[0].nbytes for b in blocks):
            raise ValueError("InputSlots: every slot's block must have the first block's size")
        self.device = device
        self.blocks = list(blocks)
        self.graphs: list = [None] * len(blocks)

    def __len__(self) -> int:
        return len(self.blocks)

    @property
    def ready(self) -> bool:
        return all(g is not None and g.live for g in self.graphs)

    def launch(self, k: int) -> None:
        """Launch slot k's graph (it reads blocks[k] as the stream reaches it)."""
        if not 0 <= k < len(self.blocks):
            raise IndexError(f"input slot {k} outside [0, {len(self.blocks)})")
        if not self.ready:
            raise RuntimeError("InputSlots.launch: a slot has no captured graph")
        self.graphs[k].replay()

    def close_extra(self) -> None:
        """Close slots 1..n-1's graphs (slot 0's is the step's own)."""
        for g in self.graphs[1:]:
            if g is not None:
                g.close()
        self.graphs = [self.graphs[0]] + [None] * (len(self.blocks) - 1)
