"""Calling a network at whatever lane count arrives, and the acting step.

Same surface as ttrl/nets/acting.py:22-188: `net_at_batch` builds a view of a
net at another batch against the same parameters (a convolution is the only
module whose shapes depend on the batch it was built for; every other module
reads the row count off its input), keeping one view module per source
module so shared trunks stay shared; `ActingNet` keeps one view per lane
count a caller actually uses and refuses a count above the width the net
was built for; `check_encoder_layout` refuses space-to-depth towers.

On top of the reference's eager `__call__`, `ActingNet.decide` runs a whole
acting step the MI355X way: per lane count, the observation (and the noise
of a stochastic policy) sits in one bound device block, the encoder forward
and the fused head-and-decision kernel (`ttrl_q_act` for a Q head,
`ttrl_gaussian_act` for a Gaussian head) are captured once into a hipGraph,
and a step is one native call (`ttrl_graph_step`): host-to-device copy of the
block, replay, device-to-host copy of a few bytes per lane, wait.  The graph
reads the master parameters in place, so it sees every optimizer update.
"""

from __future__ import annotations

import copy
import ctypes as C

import numpy as np

from ttrl_amd import _lib
from ttrl_amd.engine.autograd import Tensor, no_grad
from ttrl_amd.engine.conv import Conv2d
from ttrl_amd.engine.nn import Module
from ttrl_amd.engine.tensor import bound_block
from ttrl_amd.engine.trace import capture

__all__ = ["ActingNet", "CategoricalValueDecision", "GreedyDecision", "SquashedDecision", "check_encoder_layout",
           "net_at_batch"]

MODES = ("eager", "graph")


def _walk_modules(module, prefix: str = "net", seen: set | None = None):
    """Every Module in a tree, named by the path that reaches it
    (ttrl/nets/acting.py:47-66)."""
    seen = set() if seen is None else seen
    if not isinstance(module, Module) or id(module) in seen:
        return
    seen.add(id(module))
    yield prefix, module
    for name, child in module._slot_sources():
        if isinstance(child, dict):
            items = child.items()
        elif isinstance(child, (list, tuple)):
            items = enumerate(child)
        else:
            items = [(None, child)]
        for key, item in items:
            path = f"{prefix}.{name}" if key is None else f"{prefix}.{name}.{key}"
            yield from _walk_modules(item, path, seen)


def check_encoder_layout(net) -> None:
    """Refuse a net with a folded (space-to-depth) convolution: the acting
    buffers hold plain frames (ttrl/nets/acting.py:27-44)."""
    for name, module in _walk_modules(net):
        geom = getattr(module, "geom", None)
        if geom is not None and int(getattr(geom, "fold", 1)) != 1:
            raise ValueError(
                f"{name} is a convolution with fold={geom.fold} (space-to-depth); the acting buffers hold "
                f"plain frames, so this layer would convolve reordered pixels. Build the agent with "
                f"encoder='nature_cnn' instead of a folded tower.")


def net_at_batch(net, batch: int, _seen: dict | None = None):
    """A view of `net` taking `batch` observations, sharing its parameters
    (ttrl/nets/acting.py:69-114).  One source module becomes one view
    module, so two slots holding one object hold one view."""
    seen = {} if _seen is None else _seen
    key = id(net)
    if key in seen:
        return seen[key]
    if isinstance(net, Conv2d):
        view = net.at_batch(batch)
    elif isinstance(net, dict):
        view = {k: net_at_batch(v, batch, seen) for k, v in net.items()}
    elif isinstance(net, (list, tuple)):
        view = type(net)(net_at_batch(child, batch, seen) for child in net)
    elif not isinstance(net, Module):
        return net
    else:
        view = copy.copy(net)
        # Recorded before the children are walked, so a module reachable from
        # its own subtree resolves to this view.
        seen[key] = view
        for name, value in vars(net).items():
            setattr(view, name, net_at_batch(value, batch, seen))
        return view
    seen[key] = view
    return view


class GreedyDecision:
    """A Q network's decision: the first-index argmax of its last Linear
    layer's row (the network is EncoderHead(encoder, QHead))."""

    kind = "greedy"

    def outputs(self, net, lanes: int):
        A = _q_layer(net).out_features
        return [("actions", np.zeros(lanes, np.int32)), ("q", np.zeros((lanes, A), np.float32))]

    def inputs(self, net, lanes: int):
        return []

    def launch(self, dev, net, features: Tensor, ins, outs, deterministic: bool) -> None:
        lin = _q_layer(net)
        L, K = (int(d) for d in features.shape)
        w = lin.effective_weight()
        dev.call("ttrl_q_act", L, K, lin.out_features, features.data.ptr, w.data.ptr,
                 None if lin.bias is None else lin.bias.data.ptr, outs["q"].ptr, outs["actions"].ptr)


class SquashedDecision:
    """A Gaussian policy's decision: the tanh-squashed sample at host-drawn
    noise, or tanh(mean) when deterministic, mapped onto the action bounds
    by `scale` (an ActionScale constructed with the device)."""

    kind = "squashed"

    def __init__(self, scale):
        if getattr(scale, "_scale", None) is None:
            raise ValueError("SquashedDecision needs an ActionScale built with a device")
        self.scale = scale

    def outputs(self, net, lanes: int):
        d = net.head.action_dim
        return [("action", np.zeros((lanes, d), np.float32)), ("logp", np.zeros(lanes, np.float32))]

    def inputs(self, net, lanes: int):
        return [("noise", np.zeros((lanes, net.head.action_dim), np.float32))]

    def launch(self, dev, net, features: Tensor, ins, outs, deterministic: bool) -> None:
        head = net.head
        lm, ls = head.heads["mean"], head.heads["log_std"]
        L, K = (int(d) for d in features.shape)
        s = self.scale
        dev.call("ttrl_gaussian_act", L, K, head.action_dim, features.data.ptr, lm.weight.data.ptr,
                 None if lm.bias is None else lm.bias.data.ptr, ls.weight.data.ptr,
                 None if ls.bias is None else ls.bias.data.ptr, C.c_float(head.log_std_min),
                 C.c_float(head.log_std_max), ins["noise"].ptr, s._centre.data.ptr, s._scale.data.ptr,
                 C.c_float(s.log_det), int(deterministic), None, outs["action"].ptr, outs["logp"].ptr)


class CategoricalValueDecision:
    """A shared-trunk actor-critic's acting outputs: the log-softmax of the
    policy logits and the critic's value, per lane, computed on the device
    (the categorical draw is made on the host from these, as
    ttrl/algos/ppo/policy.py:37-62 does, and the log-prob recorded for the
    importance ratio is read from the same rows)."""

    kind = "categorical"

    def features(self, net, obs: Tensor) -> Tensor:
        return net.encoders["actor"](obs)

    def outputs(self, net, lanes: int):
        A = net.heads["policy"].logits.out_features
        return [("logp", np.zeros((lanes, A), np.float32)), ("value", np.zeros((lanes, 1), np.float32))]

    def inputs(self, net, lanes: int):
        return []

    def launch(self, dev, net, features: Tensor, ins, outs, deterministic: bool) -> None:
        from ttrl_amd.engine.ops import _kernels as K
        from ttrl_amd.engine.ops.functional import log_softmax
        from ttrl_amd.engine.tensor import DeviceArray
        from ttrl_amd.nets.heads import policy_value_packed

        L = int(features.shape[0])
        A = outs["logp"].shape[1]
        with no_grad():
            head = policy_value_packed(net.heads["policy"], net.heads["value"], features).data
            logits = DeviceArray(dev, (L, A))
            K.copy_region(head, (0, 0), logits, (0, 0), (L, A))
            logp = log_softmax(Tensor(logits), dim=-1).data
        K.copy_region(logp, (0, 0), outs["logp"], (0, 0), (L, A))
        K.copy_region(head, (0, A), outs["value"], (0, 0), (L, 1))


def _q_layer(net):
    head = getattr(net, "head", None)
    lin = getattr(head, "q", None)
    if lin is None or not hasattr(lin, "out_features"):
        raise ValueError("GreedyDecision needs an EncoderHead whose head is a QHead")
    return lin


class _Width:
    """One lane count: the view, its bound input and output blocks, and its
    captured acting graphs (one per `deterministic` value)."""

    def __init__(self, acting: "ActingNet", lanes: int):
        dev = acting.device
        self.lanes = lanes
        self.net = acting._net if lanes == acting.width else net_at_batch(acting._net, lanes)
        spec = acting.obs_spec
        if spec.kind == "image":
            host_obs = np.zeros((lanes,) + tuple(spec.shape), np.uint8)
        else:
            host_obs = np.zeros((lanes, spec.size), np.float32)
        dec = acting.decision
        ins = [("obs", host_obs)] + (dec.inputs(self.net, lanes) if dec is not None else [])
        # mapped: the blocks are pinned host memory the kernels read and write
        # in place, and in_host / out_host are their host views
        self.mapped = acting.mapped
        self.ins, self.in_block = bound_block(dev, ins, mapped=self.mapped)
        self.obs = Tensor(self.ins["obs"])
        self.outs, self.out_block = (bound_block(dev, dec.outputs(self.net, lanes), mapped=self.mapped)
                                     if dec is not None else ({}, None))
        if self.mapped:
            self.in_host = self.in_block.block.host.array[:self.in_block.nbytes]
            self.out_host = (self.out_block.block.host.array[:self.out_block.nbytes] if self.out_block is not None
                             else np.zeros(0, np.uint8))
        else:
            self.in_host = np.zeros(self.in_block.nbytes, np.uint8)
            self.out_host = np.zeros(self.out_block.nbytes if self.out_block is not None else 0, np.uint8)
        self.graphs: dict = {}
        self.pool = None

    def stage(self, name: str, array) -> None:
        """Place one input in the host image of the input block."""
        view = self.ins[name]
        arr = np.ascontiguousarray(array)
        if arr.dtype != view.dtype or arr.size != view.numel:
            raise ValueError(f"acting input {name!r}: {arr.dtype}{arr.shape} does not fit the bound "
                             f"{view.dtype}{view.shape}")
        off = view.offset - self.in_block.offset
        self.in_host[off:off + arr.nbytes] = arr.reshape(-1).view(np.uint8)

    def read(self) -> dict:
        out = {}
        for name, view in self.outs.items():
            off = view.offset - self.out_block.offset
            out[name] = self.out_host[off:off + view.nbytes].view(view.dtype).reshape(view.shape).copy()
        return out

    def close(self, dev) -> None:
        for g in self.graphs.values():
            g.close()
        self.graphs.clear()
        if self.pool is not None and not dev.closed:
            dev.release_pool(self.pool)
        self.pool = None


class ActingNet:
    """A net called at whatever lane count arrives (ttrl/nets/acting.py:117-188).

    `width` is the batch the net was built for and the widest call accepted.
    `decision` (GreedyDecision / SquashedDecision, or None) enables
    `decide`; `mode` is "graph" (captured acting step) or "eager".  With
    `direct` (the default) a captured step replays its few kernels as
    individual launches (`CapturedTrace.set_direct`): one step waits for its
    result, and a graph launch's fixed cost exceeds the launches of a handful
    of kernels.  With `mapped` (the default) the step's input and output
    blocks are pinned host memory the kernels read and write in place, so a
    step is the launches and one wait, with no copy either way.
    """

    def __init__(self, net, obs_spec, device, *, width: int, lanes: int, decision=None, mode: str = "graph",
                 direct: bool = True, mapped: bool = True):
        if mode not in MODES:
            raise ValueError(f"ActingNet mode must be one of {list(MODES)}, got {mode!r}")
        check_encoder_layout(net)
        self.obs_spec = obs_spec
        self.device = device
        self.width = int(width)
        self.decision = decision
        self.mode = mode
        self.direct = bool(direct)
        self.mapped = bool(mapped)
        self._net = net
        self._views: dict[int, _Width] = {}
        self._view(int(lanes))

    def _view(self, lanes: int) -> _Width:
        if lanes < 1:
            raise ValueError(f"ActingNet: need at least one observation, got {lanes}")
        if lanes > self.width:
            raise ValueError(
                f"ActingNet was built for at most {self.width} observations and was given {lanes}. A "
                f"convolution fixes its batch at construction, so raise the network batch to at least "
                f"{lanes} or run fewer environments.")
        w = self._views.get(lanes)
        if w is None:
            w = self._views[lanes] = _Width(self, lanes)
        return w

    def _lanes_of(self, obs) -> tuple[int, np.ndarray]:
        arr = np.asarray(obs)
        spec = self.obs_spec
        leaf = tuple(spec.shape) if spec.kind == "image" else (spec.size,)
        if arr.ndim != len(leaf) + 1 or tuple(arr.shape[1:]) != leaf:
            raise ValueError(f"ActingNet: observations must be (lanes, {', '.join(map(str, leaf))}), "
                             f"got {arr.shape}")
        if spec.kind == "image":
            if arr.dtype != np.uint8:
                raise ValueError(f"ActingNet: image observations are uint8 frames, got {arr.dtype}")
        else:
            arr = arr.astype(np.float32, copy=False)
        return int(arr.shape[0]), arr

    def __call__(self, obs, *args, **kwargs):
        """Eager forward at the lane count of `obs` (no tape)."""
        lanes, arr = self._lanes_of(obs)
        w = self._view(lanes)
        w.obs.data.upload(arr)
        with no_grad():
            return w.net(w.obs, *args, **kwargs)

    def step(self, obs, *args, **kwargs):
        """A recurrent net's single-timestep entry; a feedforward net has none."""
        lanes, arr = self._lanes_of(obs)
        w = self._view(lanes)
        fn = getattr(w.net, "step", None)
        if fn is None:
            raise TypeError(f"{type(w.net).__name__} has no single-timestep `step`; only a recurrent network "
                            f"carries state from one acting step to the next")
        w.obs.data.upload(arr)
        with no_grad():
            return fn(w.obs, *args, **kwargs)

    # -- the acting step -----------------------------------------------------

    def _body(self, w: _Width, deterministic: bool) -> None:
        encode = getattr(self.decision, "features", None)
        with no_grad():
            features = encode(w.net, w.obs) if encode is not None else w.net.encoder(w.obs)
        self.decision.launch(self.device, w.net, features, w.ins, w.outs, deterministic)

    def _graph(self, w: _Width, deterministic: bool):
        g = w.graphs.get(deterministic)
        if g is None:
            dev = self.device
            if w.pool is None:
                w.pool = dev.create_pool()
            with dev.use_pool(w.pool):
                self._body(w, deterministic)  # warm-up: tunes plans and fills the pool's free lists
                dev.synchronize()
                g, _ = capture(dev, lambda: self._body(w, deterministic))
            if self.direct:
                g.set_direct(True)
            w.graphs[deterministic] = g
        return g

    def decide(self, obs, *, noise=None, deterministic: bool = False) -> dict:
        """One acting step: {"actions", "q"} for a greedy decision,
        {"action", "logp"} for a squashed one, {"logp" (lanes, A), "value"}
        for a categorical one, as host arrays."""
        if self.decision is None:
            raise TypeError("ActingNet.decide needs a decision (GreedyDecision or SquashedDecision)")
        lanes, arr = self._lanes_of(obs)
        w = self._view(lanes)
        w.stage("obs", arr)
        if "noise" in w.ins:
            if noise is None:
                if not deterministic:
                    raise ValueError("ActingNet.decide: a stochastic squashed step needs noise")
            else:
                w.stage("noise", np.asarray(noise, np.float32).reshape(w.ins["noise"].shape))
        dev = self.device
        lib = _lib.lib()
        in_ptr, out_ptr = C.c_void_p(w.in_block.ptr), C.c_void_p(w.out_block.ptr)
        host_in = w.in_host.ctypes.data_as(C.c_void_p)
        host_out = w.out_host.ctypes.data_as(C.c_void_p)
        if w.mapped:
            # the kernels read the staged inputs and write the outputs in place
            if self.mode == "graph":
                g = self._graph(w, bool(deterministic))
                _lib.check(lib.ttrl_graph_step(dev.ctx, g._graph, None, None, 0, None, None, 0), "ttrl_graph_step")
            else:
                self._body(w, bool(deterministic))
                dev.synchronize()
        elif self.mode == "graph":
            g = self._graph(w, bool(deterministic))
            _lib.check(lib.ttrl_graph_step(dev.ctx, g._graph, in_ptr, host_in, w.in_host.nbytes, host_out,
                                           out_ptr, w.out_host.nbytes), "ttrl_graph_step")
        else:
            _lib.check(lib.ttrl_graph_step(dev.ctx, None, in_ptr, host_in, w.in_host.nbytes, None, None, 0),
                       "ttrl_graph_step")
            self._body(w, bool(deterministic))
            _lib.check(lib.ttrl_graph_step(dev.ctx, None, None, None, 0, host_out, out_ptr, w.out_host.nbytes),
                       "ttrl_graph_step")
        return w.read()

    def close(self) -> None:
        """Release every width's graphs and pools.  Idempotent."""
        for w in self._views.values():
            w.close(self.device)
        self._views.clear()
