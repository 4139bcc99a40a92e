"""Host bookkeeping of input slots (ttrl_amd.engine.slots), without a GPU:
the twin block's input views, slot launches, and the argument checks."""

from __future__ import annotations

import numpy as np
import pytest


class _Dev:
    """Hands out fake addresses and records the library calls."""

    closed = False

    def __init__(self):
        self.next = 1 << 20
        self.calls = []

    def alloc(self, nbytes):
        p = self.next
        self.next += (int(nbytes) + 255) // 256 * 256 + 4096
        return p

    def free(self, ptr):
        pass

    def call(self, name, *args):
        self.calls.append((name, args))

    def host_block(self, nbytes):
        return _HostImage(nbytes)


class _HostImage:
    def __init__(self, nbytes):
        self.buf = np.zeros(int(nbytes), np.uint8)
        self.nbytes = int(nbytes)
        self.ptr = self.buf.ctypes.data

    def view(self, off, shape, dtype):
        n = int(np.prod(shape)) * np.dtype(dtype).itemsize
        return self.buf[off:off + n].view(dtype).reshape(shape)

    def close(self):
        pass


class _Graph:
    def __init__(self, log, tag):
        self.log, self.tag, self.live = log, tag, True

    def replay(self):
        self.log.append(self.tag)

    def close(self):
        self.live = False


def _inputs(dev):
    from ttrl_amd.engine.autograd import Tensor
    from ttrl_amd.engine.tensor import DeviceArray, _Block

    blk = _Block(dev, 4096)
    whole = DeviceArray(dev, (4096,), np.uint8, block=blk)
    obs = DeviceArray(dev, (2, 8), np.uint8, block=blk, offset=0)
    rew = DeviceArray(dev, (2, 1), np.float32, block=blk, offset=256)
    outside = DeviceArray(dev, (3,), np.float32)
    return {"_block": whole, "obs": Tensor(obs), "rewards": Tensor(rew), "table": Tensor(outside)}


def test_twin_inputs_mirror_the_block_layout():
    from ttrl_amd.engine.slots import twin_inputs

    dev = _Dev()
    inputs = _inputs(dev)
    twin = twin_inputs(dev, inputs)
    assert twin["_block"].block is not inputs["_block"].block
    assert twin["_block"].nbytes == inputs["_block"].nbytes
    for name in ("obs", "rewards"):
        a, b = inputs[name].data, twin[name].data
        assert b.block is twin["_block"].block
        assert (b.offset, b.shape, b.dtype) == (a.offset, a.shape, a.dtype)
        assert b.ptr - twin["_block"].ptr == a.ptr - inputs["_block"].ptr
    assert twin["table"] is inputs["table"]  # not part of the block: shared


def test_slot_launch_runs_that_slots_graph():
    from ttrl_amd.engine.slots import InputSlots, twin_inputs

    dev = _Dev()
    inputs = _inputs(dev)
    slots = InputSlots(dev, [inputs["_block"]] + [twin_inputs(dev, inputs)["_block"] for _ in range(2)])
    with pytest.raises(RuntimeError, match="no captured graph"):
        slots.launch(0)
    log = []
    slots.graphs = [_Graph(log, k) for k in range(3)]
    for k in (2, 0, 1, 1):
        slots.launch(k)
    assert log == [2, 0, 1, 1]
    with pytest.raises(IndexError, match="outside"):
        slots.launch(3)
    first = slots.graphs[0]
    slots.close_extra()
    assert first.live and slots.graphs[0] is first and slots.graphs[1:] == [None, None]


def test_input_slots_refuse_bad_layouts():
    from ttrl_amd.engine.slots import MAX_SLOTS, InputSlots
    from ttrl_amd.engine.tensor import DeviceArray

    dev = _Dev()
    a = DeviceArray(dev, (4096,), np.uint8)
    with pytest.raises(ValueError, match="between 2 and"):
        InputSlots(dev, [a])
    with pytest.raises(ValueError, match="between 2 and"):
        InputSlots(dev, [a] * (MAX_SLOTS + 1))
    with pytest.raises(ValueError, match="first block's size"):
        InputSlots(dev, [a, DeviceArray(dev, (2048,), np.uint8)])


def test_train_step_slots_need_graph_mode_and_a_bound_block():
    from ttrl_amd.engine.step import TrainStep

    dev = _Dev()
    eager = TrainStep(lambda inputs: {}, {}, dev, mode="eager")
    with pytest.raises(ValueError, match="mode='graph'"):
        eager.enable_input_slots(2)
    loose = TrainStep(lambda inputs: {}, {}, dev, mode="graph")
    with pytest.raises(ValueError, match="one bound block"):
        loose.enable_input_slots(2)
    with pytest.raises(RuntimeError, match="enable_input_slots"):
        loose.replay_slot(0)
    bound = TrainStep(lambda inputs: {}, _inputs(dev), dev, mode="graph")
    with pytest.raises(ValueError, match="between 2 and"):
        bound.enable_input_slots(1)
    bound.enable_input_slots(3)
    assert bound.slot_inputs(0) is bound.inputs
    assert bound.slot_inputs(2)["_block"].nbytes == bound.inputs["_block"].nbytes
    with pytest.raises(RuntimeError, match="once"):
        bound.enable_input_slots(2)
    with pytest.raises(RuntimeError, match="run\\(\\) once first"):
        bound.replay_slot(1)


def test_binder_queues_large_inputs_and_waits_before_restaging_them(monkeypatch):
    """InputBinder.load: an input of at least QUEUE_MIN_BYTES is queued as
    soon as it is staged (ttrl_h2d_enqueue) and leaves the pending ranges;
    staging it again first waits for the stream; a flush or graph step that
    waits clears that; small inputs stay pending for the one batch copy."""
    from ttrl_amd.engine.step import InputBinder

    dev = _Dev()
    dev.capturing = False
    dev.synchronize = lambda: dev.calls.append(("sync", ()))
    inputs = _inputs(dev)
    binder = InputBinder(dev, inputs)
    monkeypatch.setattr(InputBinder, "QUEUE_MIN_BYTES", 16)  # obs: 16 bytes, rewards: 8
    binder.load("obs", np.arange(16, dtype=np.uint8).reshape(2, 8))
    assert [c[0] for c in dev.calls] == ["ttrl_h2d_enqueue"]
    dst, src, n = (a.value for a in dev.calls[0][1])
    assert (dst, src, n) == (inputs["_block"].ptr, binder.image.ptr, 16)
    assert np.array_equal(binder.image.buf[:16], np.arange(16))
    assert binder.pending() == []
    binder.load("rewards", np.ones((2, 1), np.float32))
    assert binder.pending() == [(256, 264)] and len(dev.calls) == 1
    binder.load("obs", np.zeros((2, 8), np.uint8))  # its queued copy may still read the image
    assert [c[0] for c in dev.calls] == ["ttrl_h2d_enqueue", "sync", "ttrl_h2d_enqueue"]
    binder.flush()  # ttrl_h2d waits for the stream
    assert dev.calls[-1][0] == "ttrl_h2d" and binder.pending() == []
    binder.load("obs", np.ones((2, 8), np.uint8))
    assert [c[0] for c in dev.calls[-2:]] == ["ttrl_h2d", "ttrl_h2d_enqueue"]
    binder.synced()
    binder.load("obs", np.ones((2, 8), np.uint8))
    assert "sync" not in [c[0] for c in dev.calls[-2:]]
    dev.capturing = True  # never queued during a capture
    binder.synced()
    binder.load("obs", np.ones((2, 8), np.uint8))
    assert dev.calls[-1][0] == "ttrl_h2d_enqueue" and binder.pending() == [(0, 16)]
