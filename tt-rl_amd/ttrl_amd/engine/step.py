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
"""

from __future__ import annotations

from typing import Callable

import numpy as np

from ttrl_amd.engine.autograd import Tensor
from ttrl_amd.engine.trace import capture

__all__ = ["MODES", "StepFn", "TrainStep", "read_metrics", "InputBinder"]

StepFn = Callable[[dict], dict]

MODES = ("eager", "traced_fwd_bwd", "graph")


class InputBinder:
    """Copies fresh host data into bound input buffers, never rebinding them."""

    def __init__(self, device, inputs: dict):
        self.device = device
        self.inputs = inputs

    def load(self, name: str, array) -> None:
        t = self.inputs[name]
        arr = np.asarray(array)
        want = t.data.dtype
        if arr.dtype != want:
            arr = arr.astype(want)
        if arr.size != t.data.numel:
            raise ValueError(f"load_input({name!r}): {arr.shape} does not fit the bound buffer {t.shape}")
        t.data.upload(arr)

    def close(self) -> None:
        pass


def read_metrics(metrics: dict | None) -> dict:
    """Download every tensor-valued metric; non-tensors pass through."""
    if not metrics:
        return {}
    out = {}
    for k, v in metrics.items():
        out[k] = v.numpy() if isinstance(v, Tensor) else v
    return out


class TrainStep:
    def __init__(self, step_fn: StepFn, inputs: dict, device, *, optimizer=None, mode: str = "eager", cfg=None):
        if mode not in MODES:
            raise ValueError(f"TrainStep mode must be one of {list(MODES)}, got {mode!r}")
        self.step_fn = step_fn
        self.inputs = inputs
        self.device = device
        self.optimizer = optimizer
        self.mode = mode
        self.cfg = cfg
        self._binder = InputBinder(device, inputs)
        self._trace = None
        self._trace_metrics: dict | None = None
        self._captured_grads: list = []
        self._pool = None

    def load_input(self, name: str, array) -> None:
        self._binder.load(name, array)

    def run(self) -> dict:
        if self.mode == "eager":
            return self._run_eager()
        return self._run_graph()

    def _run_eager(self) -> dict:
        if self.optimizer is not None:
            self.optimizer.zero_grad()
        metrics = self.step_fn(self.inputs)
        if self.optimizer is not None:
            self.optimizer.step()
        return read_metrics(metrics)

    def replay(self) -> None:
        """Launch the captured step without reading metrics (benchmark loop)."""
        self._trace.replay()
        self._rebind_grads()
        if self.optimizer is not None:
            if self.mode == "graph":
                self.optimizer._replayed()
            else:
                self.optimizer.step()

    def _run_graph(self) -> dict:
        if self._trace is None:
            self._capture()
        else:
            self.replay()
        return read_metrics(self._trace_metrics)

    def _body(self, with_optimizer: bool):
        metrics = self.step_fn(self.inputs)
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
        if self.optimizer is not None:
            self._captured_grads = [(p, p.grad) for p in self.optimizer.params]
        self._trace.replay(blocking=True)
        if self.optimizer is not None:
            if in_graph:
                self.optimizer._replayed()
            else:
                self.optimizer.step()

    def _rebind_grads(self) -> None:
        for param, grad in self._captured_grads:
            param.grad = grad

    def close(self) -> None:
        trace, self._trace = self._trace, None
        self._trace_metrics = None
        self._captured_grads = []
        try:
            if trace is not None:
                trace.close()
        finally:
            self._binder.close()
            if self._pool is not None and not self.device.closed:
                self.device.release_pool(self._pool)
            self._pool = None

    def __enter__(self) -> "TrainStep":
        return self

    def __exit__(self, *exc) -> None:
        self.close()
