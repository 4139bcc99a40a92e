"""TrainStep: one training step run eagerly or replayed from a hipGraph
(replaces ttrl/engine/step/core.py:21-160, step/inputs.py:16-102,
step/metrics.py:22-112).

Modes:
  "eager"           step_fn, then the optimizer, every call;
  "traced_fwd_bwd"  the reference's trace mode: forward and backward are
                    captured once and replayed, the optimizer runs eagerly;
  "graph"           forward, backward AND the optimizer in one graph.  The
                    Adam kernel reads its update count from the device, so
                    the bias correction the reference keeps out of its trace
                    for (core.py:35-41) is correct on every replay.

The first call captures: a warm-up pass (real dispatch, gradients discarded)
populates the step's private allocation pool so the capture pass reuses the
same blocks, then the capture, then one replay so the call returns this
step's metrics.  Buffers the graph touches come from that pool and stay
reserved for the graph's lifetime.

With input slots (`enable_input_slots`, engine.slots) the first call
captures one graph per bound input block, and `replay_slot(k)` runs the
update on the batch written into slot k's block.
"""

from __future__ import annotations

from typing import Callable

import ctypes as C

import numpy as np

from ttrl_amd.engine.autograd import Tensor
from ttrl_amd.engine.config import DEFAULT, EngineConfig, check_engine_config
from ttrl_amd.engine.pending import take_sources
from ttrl_amd.engine.slots import InputSlots, check_slot_count, metric_ptrs, twin_inputs
from ttrl_amd.engine.tensor import DeviceArray
from ttrl_amd.engine.trace import capture

__all__ = ["MODES", "StepFn", "TrainStep", "read_metrics", "InputBinder", "MetricReader"]

StepFn = Callable[[dict], dict]

MODES = ("eager", "traced_fwd_bwd", "graph")


class InputBinder:
    """Writes fresh host data into the bound input buffers, never rebinding
    them (ttrl/engine/step/inputs.py:16-102).

    Inputs that are views of one bound block (`inputs["_block"]`, laid out
    by `bound_block`) are staged in a pinned host image of that block:
    `load` writes into the image only, and `flush` sends every range loaded
    since the last flush, adjacent ranges coalesced, so a full batch is one
    host-to-device copy.  An input of at least QUEUE_MIN_BYTES is instead
    queued on the stream as soon as it is staged (ttrl_h2d_enqueue), so its
    copy overlaps the staging of the inputs after it; its part of the image
    is not written again before the stream has been waited for.  Ranges not
    loaded are never sent, so device-side writes into the block (a replay
    draw assembling a batch in place) are not overwritten by stale host
    data.  Other inputs upload directly."""

    QUEUE_MIN_BYTES = 256 << 10

    def __init__(self, device, inputs: dict):
        self.device = device
        self.inputs = inputs
        self.block = inputs.get("_block")
        self.image = None
        self._views: dict = {}
        self._ranges: dict = {}
        self._dirty: set = set()
        self._queued: set = set()  # inputs whose queued copy may still read the image
        if self.block is not None and isinstance(self.block, DeviceArray):
            self.image = device.host_block(self.block.nbytes)
            for name, t in inputs.items():
                d = getattr(t, "data", None)
                if name.startswith("_") or not isinstance(d, DeviceArray) or not d.same_storage(self.block):
                    continue
                off = d.offset - self.block.offset
                self._views[name] = self.image.view(off, d.shape, d.dtype)
                self._ranges[name] = (off, off + d.nbytes)

    def load(self, name: str, array) -> None:
        t = self.inputs[name]
        arr = np.asarray(array)
        if arr.size != t.data.numel:
            raise ValueError(f"load_input({name!r}): {arr.shape} does not fit the bound buffer {t.shape}")
        view = self._views.get(name)
        if view is None:
            t.data.upload(arr.astype(t.data.dtype, copy=False))
            return
        if name in self._queued:
            self.device.synchronize()
            self._queued.clear()
        np.copyto(view, arr.reshape(view.shape), casting="unsafe")
        b, e = self._ranges[name]
        if e - b >= self.QUEUE_MIN_BYTES and not self.device.capturing:
            self.device.call("ttrl_h2d_enqueue", C.c_void_p(self.block.ptr + b), C.c_void_p(self.image.ptr + b),
                             C.c_size_t(e - b))
            self._queued.add(name)
            self._dirty.discard(name)
        else:
            self._dirty.add(name)

    def synced(self) -> None:
        """The stream has been waited for since the last load: every queued
        copy has finished reading the image."""
        self._queued.clear()

    def pending(self) -> list:
        """[(begin, end)] byte ranges of the block loaded since the last
        flush, adjacent or overlapping ranges merged."""
        spans = sorted(self._ranges[n] for n in self._dirty)
        out: list = []
        for b, e in spans:
            # bound_block starts every input on a 256-byte boundary: bridge
            # only the alignment padding after the previous range, never an
            # input that was not loaded
            if out and b <= -(-out[-1][1] // 256) * 256:
                out[-1] = (out[-1][0], max(out[-1][1], e))
            else:
                out.append((b, e))
        return out

    def flush(self) -> None:
        spans = self.pending()
        for b, e in spans:
            self.device.call("ttrl_h2d", C.c_void_p(self.block.ptr + b), C.c_void_p(self.image.ptr + b),
                             C.c_size_t(e - b))
        self._dirty.clear()
        if spans:  # ttrl_h2d waits for the stream
            self._queued.clear()

    def take_single_range(self):
        """The one pending range (begin, end) when at most one is pending
        ((0, 0) when none is), clearing
        it (the caller sends it), else None."""
        spans = self.pending()
        if not spans:
            return (0, 0)
        if len(spans) != 1:
            return None
        self._dirty.clear()
        return spans[0]

    def close(self) -> None:
        if self.image is not None:
            self.image.close()
            self.image = None
            self._views.clear()


class MetricReader:
    """Reads a step's metrics (ttrl/engine/step/metrics.py:22-112).

    When every tensor metric is a view of one device allocation, one copy of
    the span covering them lands in a pinned host image and each metric is
    sliced out of it; otherwise each tensor is read on its own."""

    def __init__(self, device):
        self.device = device
        self.image = None
        self.span = None  # (device ptr, nbytes, {name: (offset, shape, dtype)})

    def bind(self, metrics: dict | None):
        self.span = None
        tensors = {k: v.data for k, v in (metrics or {}).items() if isinstance(v, Tensor)}
        if not tensors:
            return
        arrays = list(tensors.values())
        block = arrays[0].block
        if any(a.block is not block for a in arrays):
            return
        lo = min(a.ptr for a in arrays)
        hi = max(a.ptr + a.nbytes for a in arrays)
        if self.image is None or self.image.nbytes < hi - lo:
            if self.image is not None:
                self.image.close()
            self.image = self.device.host_block(hi - lo)
        self.span = (lo, hi - lo, {k: (a.ptr - lo, a.shape, a.dtype) for k, a in tensors.items()})

    def _unpack(self, metrics: dict) -> dict:
        ptr, n, layout = self.span
        out = {}
        for k, v in metrics.items():
            if k in layout:
                off, shape, dtype = layout[k]
                out[k] = self.image.view(off, shape, dtype).copy()
            else:
                out[k] = v
        return out

    def read(self, metrics: dict | None) -> dict:
        if not metrics:
            return {}
        if self.span is None:
            return read_metrics(metrics)
        ptr, n, _ = self.span
        self.device.call("ttrl_d2h", C.c_void_p(self.image.ptr), C.c_void_p(ptr), C.c_size_t(n))
        return self._unpack(metrics)

    def close(self) -> None:
        if self.image is not None:
            self.image.close()
            self.image = None
        self.span = None


def read_metrics(metrics: dict | None) -> dict:
    """Download every tensor-valued metric; non-tensors pass through."""
    if not metrics:
        return {}
    out = {}
    for k, v in metrics.items():
        out[k] = v.numpy() if isinstance(v, Tensor) else v
    return out


class TrainStep:
    def __init__(self, step_fn: StepFn, inputs: dict, device, *, optimizer=None, mode: str = "eager",
                 cfg: EngineConfig = DEFAULT):
        if mode not in MODES:
            raise ValueError(f"TrainStep mode must be one of {list(MODES)}, got {mode!r}")
        self.step_fn = step_fn
        self.inputs = inputs
        self.device = device
        self.optimizer = optimizer
        self.mode = mode
        # trace_blocking: a replay waits for the device before returning
        # (ttrl/engine/step/core.py:87-91); the metric read-back waits anyway.
        self.cfg = check_engine_config(cfg, "TrainStep")
        self._binder = InputBinder(device, inputs)
        self._reader = MetricReader(device)
        self._trace = None
        self._trace_metrics: dict | None = None
        self._captured_grads: list = []
        # traced_fwd_bwd: the gradient sources and ordered sums the captured
        # backward leaves for the eager optimizer step, re-queued after
        # every replay (the replay refreshes their operands, not the host
        # records the step consumes)
        self._captured_pending: tuple = ((), ())
        self._pool = None
        self._slots: InputSlots | None = None
        self._slot_inputs: list = []
        self._slot_grads: list = []

    def enable_input_slots(self, n: int) -> None:
        """n bound input blocks of the inputs' layout (slot 0 is
        `inputs["_block"]`), one graph captured against each at the first
        run (engine.slots); `slot_inputs(k)` are slot k's input tensors and
        `replay_slot(k)` runs the update on them.  Graph mode, before the
        first run; every metric must be written to fixed buffers."""
        if self.mode != "graph":
            raise ValueError("TrainStep.enable_input_slots: input slots need mode='graph'")
        if self._trace is not None or self._slots is not None:
            raise RuntimeError("TrainStep.enable_input_slots: call it once, before the first run (the capture)")
        if not isinstance(self.inputs.get("_block"), DeviceArray):
            raise ValueError("TrainStep.enable_input_slots: the inputs must be views of one bound block (`_block`)")
        check_slot_count("TrainStep.enable_input_slots", n)
        self._slot_inputs = [self.inputs] + [twin_inputs(self.device, self.inputs) for _ in range(n - 1)]
        self._slots = InputSlots(self.device, [d["_block"] for d in self._slot_inputs])

    def slot_inputs(self, k: int) -> dict:
        """Slot k's input tensors (`_block`: its whole block)."""
        if self._slots is None:
            raise RuntimeError("TrainStep.slot_inputs: call enable_input_slots() first")
        return self._slot_inputs[k]

    def replay_slot(self, k: int) -> None:
        """Launch the captured step on slot k's inputs without reading
        metrics; they are read as after `replay()`."""
        if self._slots is None:
            raise RuntimeError("TrainStep.replay_slot: call enable_input_slots() before the first run")
        if self._trace is None:
            raise RuntimeError("TrainStep.replay_slot: run() once first (it captures every slot's graph)")
        self._slots.launch(k)
        if self.cfg.trace_blocking:
            self.device.synchronize()
            self._binder.synced()
        self._captured_grads = self._slot_grads[k]
        self._after_replay()

    def run_slot(self, k: int) -> dict:
        """Slot k's update with its metrics read back: one ttrl_graph_step
        that replays slot k's graph on the batch already in slot k's block,
        copies the packed metric span to the host and waits once."""
        if self._slots is None:
            raise RuntimeError("TrainStep.run_slot: call enable_input_slots() before the first run")
        if self._trace is None:
            raise RuntimeError("TrainStep.run_slot: run() once first (it captures every slot's graph)")
        span = self._reader.span
        if span is None:
            self.replay_slot(k)
            return self._reader.read(self._trace_metrics)
        if not 0 <= k < len(self._slots.blocks):
            raise IndexError(f"input slot {k} outside [0, {len(self._slots.blocks)})")
        ptr, n, _ = span
        self.device.call("ttrl_graph_step", self._slots.graphs[k]._graph, None, None, C.c_size_t(0),
                         C.c_void_p(self._reader.image.ptr), C.c_void_p(ptr), C.c_size_t(n))
        self._binder.synced()
        self._captured_grads = self._slot_grads[k]
        self._after_replay()
        return self._reader._unpack(self._trace_metrics)

    def load_input(self, name: str, array) -> None:
        self._binder.load(name, array)

    def flush_inputs(self) -> None:
        """Send staged inputs now (the next run would send them anyway)."""
        self._binder.flush()

    def run(self) -> dict:
        if self.mode == "eager":
            return self._run_eager()
        return self._run_graph()

    def _run_eager(self) -> dict:
        self._binder.flush()
        if self.optimizer is not None:
            self.optimizer.zero_grad()
        metrics = self.step_fn(self.inputs)
        if self.optimizer is not None:
            self.optimizer.step()
        self._reader.bind(metrics)
        return self._reader.read(metrics)

    def replay(self) -> None:
        """Launch the captured step without reading metrics (benchmark loop);
        with `cfg.trace_blocking` it returns once the device has finished."""
        self._binder.flush()
        self._trace.replay(blocking=self.cfg.trace_blocking)
        if self.cfg.trace_blocking:
            self._binder.synced()
        self._after_replay()

    def _after_replay(self) -> None:
        self._rebind_grads()
        if self.optimizer is not None:
            if self.mode == "graph":
                self.optimizer._replayed()
            else:
                self._requeue_pending()
                self.optimizer.step()

    def _requeue_pending(self) -> None:
        """Re-attach the captured backward's pending gradient sources to
        their tensors and queue its ordered sums again, so the eager step
        after this replay forms them from the operands the replay wrote."""
        sources, sums = self._captured_pending
        for pend in sources:
            for t in pend.tensors:
                t._pending = pend
        queued = self.device.pending_sums
        for item in sums:
            if all(item is not q for q in queued):
                queued.append(item)

    def _run_graph(self) -> dict:
        if self._trace is None:
            self._binder.flush()
            self._capture()
            self._reader.bind(self._trace_metrics)
            return self._reader.read(self._trace_metrics)
        span = self._reader.span
        sent = self._binder.take_single_range() if (span is not None and self.mode == "graph") else None
        if sent is None:
            self.replay()
            if not self._trace_metrics and not self.cfg.trace_blocking:
                # nothing to read back orders the replay ahead of the caller's
                # next host step (ttrl/engine/step/core.py:135-141)
                self.device.synchronize()
                self._binder.synced()
            return self._reader.read(self._trace_metrics)
        # One call: the loaded input range in, the replay, the metric span out, one wait.
        b, e = sent
        blk, img = self._binder.block, self._binder.image
        ptr, n, _ = span
        self.device.call("ttrl_graph_step", self._trace._graph, C.c_void_p(blk.ptr + b), C.c_void_p(img.ptr + b),
                         C.c_size_t(e - b), C.c_void_p(self._reader.image.ptr), C.c_void_p(ptr), C.c_size_t(n))
        self._binder.synced()  # ttrl_graph_step waits for the stream
        self._after_replay()
        return self._reader._unpack(self._trace_metrics)

    def _body(self, with_optimizer: bool, inputs: dict | None = None):
        metrics = self.step_fn(self.inputs if inputs is None else inputs)
        if with_optimizer and self.optimizer is not None:
            self.optimizer.step()
        return metrics

    def _capture(self) -> None:
        dev = self.device
        in_graph = self.mode == "graph"
        if self._pool is None:
            self._pool = dev.create_pool()
        with dev.use_pool(self._pool):
            if self.optimizer is not None:
                self.optimizer.zero_grad()
            self.step_fn(self.inputs)  # warm-up: fills the pool's free lists
            if self.optimizer is not None:
                self.optimizer.zero_grad()
            dev.synchronize()
            self._trace, self._trace_metrics = capture(dev, lambda: self._body(in_graph))
            self._captured_grads = self._grads_now()
            if not in_graph and self.optimizer is not None:
                self._captured_pending = (tuple(take_sources(self.optimizer.params)), tuple(dev.pending_sums))
            if self._slots is not None:
                self._capture_slots(in_graph)
        self._rebind_grads()
        self._trace.replay(blocking=True)
        if self.optimizer is not None:
            if in_graph:
                self.optimizer._replayed()
            else:
                self.optimizer.step()

    def _grads_now(self) -> list:
        return [(p, p.grad) for p in self.optimizer.params] if self.optimizer is not None else []

    def _capture_slots(self, in_graph: bool) -> None:
        """Slot k >= 1's graph: the same update over slot k's inputs."""
        dev = self.device
        want = metric_ptrs(self._trace_metrics)
        self._slots.graphs[0] = self._trace
        self._slot_grads = [self._captured_grads]
        for k, inputs in enumerate(self._slot_inputs[1:], start=1):
            if self.optimizer is not None:
                self.optimizer.zero_grad()
            trace, metrics = capture(dev, lambda inputs=inputs: self._body(in_graph, inputs))
            self._slots.graphs[k] = trace
            self._slot_grads.append(self._grads_now())
            if metric_ptrs(metrics) != want:
                raise RuntimeError("TrainStep.enable_input_slots: the step's metrics are not written to the same "
                                   "buffers by every slot's graph; give the step fixed metric outputs")

    def _rebind_grads(self) -> None:
        for param, grad in self._captured_grads:
            param.grad = grad

    def close(self) -> None:
        trace, self._trace = self._trace, None
        self._trace_metrics = None
        self._captured_grads = []
        self._captured_pending = ((), ())
        slots, self._slots = self._slots, None
        try:
            if slots is not None:
                slots.close_extra()
            if trace is not None:
                trace.close()
        finally:
            self._binder.close()
            self._reader.close()
            if self._pool is not None and not self.device.closed:
                self.device.release_pool(self._pool)
            self._pool = None

    def __enter__(self) -> "TrainStep":
        return self

    def __exit__(self, *exc) -> None:
        self.close()
