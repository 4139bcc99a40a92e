"""Adam over fp32 parameters, updated in place (ttrl/engine/optim/adam.py:25-134).

Stores S = m/(1-b1) and V = v/(1-b2) like the reference, so the fused
bias-correction scalars (ttrl/engine/optim/scalars.py:13-27) apply unchanged
and checkpoints carry canonical m and v (ttrl/engine/optim/checkpoint.py:15-104).

One kernel updates a whole parameter arena (every tensor of a network built
inside one `ParamArena`), reading the update count from a device counter so
that a captured graph containing the step replays correctly for every t.
The same launch reduces sum(g^2) into `grad_sq` (ttrl/algos/grads.py:46-60).
Gradients an earlier launch left pending (engine.pending: split-K partials,
outer products) are formed by the arena step itself as it reads them, and
its finishing launch forms the ordered sums queued on the device.

Several optimizers stepped in one update (SAC's critic, actor and
temperature) can defer their finishes: `step_deferred` or one `adam_multi`
launch for several arenas (with the Polyak blend), then one `finish_steps`
launch that stores every update count and sum(g^2).
"""

from __future__ import annotations

import ctypes as C
import math

import numpy as np

from ttrl_amd import _lib
from ttrl_amd.engine.pending import MAX_SOURCES, MAX_SUMS, settle, settle_sums, take_sources, take_sums
from ttrl_amd.engine.tensor import DeviceArray, MASTER_DTYPE, arena_of, zeros

__all__ = ["Adam", "Optimizer", "adam_fused_scalars", "adam_multi", "finish_steps"]


def adam_fused_scalars(lr: float, b1: float, b2: float, eps: float, t: int) -> tuple[float, float]:
    """(alpha_t, eps_t) of the composed Adam tail for update number t."""
    if t < 1:
        raise ValueError(f"adam_fused_scalars: t must be >= 1, got {t}")
    bc1 = 1 - b1 ** t
    bc2 = 1 - b2 ** t
    c = math.sqrt((1 - b2) / bc2)
    return lr * (1 - b1) / bc1 / c, eps / c


class Optimizer:
    def __init__(self, params):
        self.params = list(params)

    def zero_grad(self) -> None:
        """Drops the gradients, and the work an abandoned update left
        pending: its gradient sources and the device's queued ordered sums
        (an update queues them and its own step consumes them)."""
        for p in self.params:
            p.zero_grad()
        if self.params:
            take_sums(self.params[0].device)


class Adam(Optimizer):
    """Adam over fp32 parameters, updated in place."""

    def __init__(self, params, lr=1e-4, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.0):
        super().__init__(params)
        if not self.params:
            raise ValueError("Adam: params is empty, so there is nothing to optimize")
        if lr <= 0:
            raise ValueError(f"Adam: lr must be > 0, got {lr}")
        b1, b2 = betas
        if not (0.0 <= b1 < 1.0 and 0.0 <= b2 < 1.0):
            raise ValueError(f"Adam: betas must be in [0, 1), got {betas}")
        if eps <= 0:
            raise ValueError(f"Adam: eps must be > 0, got {eps}")
        if weight_decay < 0:
            raise ValueError(f"Adam: weight_decay must be >= 0, got {weight_decay}")
        wrong = [i for i, p in enumerate(self.params) if p.data.dtype != MASTER_DTYPE]
        if wrong:
            raise ValueError(f"Adam: parameters must be float32; parameters {wrong} are not")
        self.lr = float(lr)
        self.b1, self.b2 = float(b1), float(b2)
        self.eps = float(eps)
        self.weight_decay = float(weight_decay)
        # Whether a step that forms pending gradient sources also writes
        # them into the gradient buffers.  Off, the parameters move the same
        # and `materialize_grads()` writes the last step's formed gradients
        # on request (from operands the next update overwrites).
        self.store_formed_grads = True
        self._formed: tuple = ()
        self.t = 0
        self.steps = [0] * len(self.params)
        dev = self.params[0].device
        self.device = dev
        self.arena = arena_of(self.params)
        n = len(self.params)
        # counters[i]: update count of parameter i; counters[n]: of the arena launch.
        self._counters = DeviceArray(dev, (n + 1,), np.int32)
        self._counters.fill(0)
        self._arena_t = 0
        self.grad_sq = zeros(dev, (1, 1))
        if self.arena is not None:
            self._m_flat = zeros(dev, (self.arena.numel,))
            self._v_flat = zeros(dev, (self.arena.numel,))
            self.m = [self._m_flat.view(off, p.shape) for p, off in zip(self.params, self.arena.offsets)]
            self.v = [self._v_flat.view(off, p.shape) for p, off in zip(self.params, self.arena.offsets)]
        else:
            self.m = [zeros(dev, p.shape) for p in self.params]
            self.v = [zeros(dev, p.shape) for p in self.params]

    @property
    def _m_scale(self) -> float:
        return 1 - self.b1

    @property
    def _v_scale(self) -> float:
        return 1 - self.b2

    def _counter(self, i: int) -> C.c_void_p:
        return C.c_void_p(self._counters.ptr + 4 * i)

    def step(self) -> None:
        """One update of every parameter that holds a gradient.

        Inside a graph capture nothing executes, so the host counters are
        advanced by `_replayed()` when the graph runs instead of here.
        """
        capturing = self.device.capturing
        if not capturing:
            self.t += 1
        have = [p.grad is not None for p in self.params]
        dev = self.device
        args = (C.c_float(self.lr), C.c_float(self.b1), C.c_float(self.b2), C.c_float(self.eps),
                C.c_float(self.weight_decay))
        counts_in_sync = all(s == self._arena_t for s in self.steps)
        if self.arena is not None and all(have) and counts_in_sync:
            for p in self.params:
                if p.grad is not p._grad_slot:
                    settle([p])
                    p._grad_slot.copy_from(p.grad)
                    p.grad = p._grad_slot
                    p._grad_owned = True
            a = self.arena
            sources = take_sources(self.params)
            sums = take_sums(dev)
            if sources or sums:
                self._step_sources(sources, sums)
            else:
                dev.call("ttrl_adam_step", a.data.vp, a.grad.vp, self._m_flat.vp, self._v_flat.vp,
                         C.c_long(a.numel), self._counter(len(self.params)), *args, self.grad_sq.vp, 0)
            if not capturing:
                self._arena_t += 1
                self.steps = [s + 1 for s in self.steps]
            return
        if dev.capturing:
            raise RuntimeError(
                "Adam.step inside a captured graph needs every parameter of one arena to hold a "
                "gradient; step this optimizer outside the capture instead."
            )
        settle(self.params)
        settle_sums(dev)
        self._counters.upload(np.asarray(self.steps + [self._arena_t], np.int32))
        first = True
        for i, p in enumerate(self.params):
            if p.grad is None:
                continue
            g = p.grad
            if p.data.numel % 4 or (p.data.ptr | g.ptr | self.m[i].ptr | self.v[i].ptr) % 16:
                # the kernel needs 16-byte aligned float4 ranges: stage through aligned copies
                g = _aligned_copy(g)
            self._step_one(i, p, g, args, accumulate=not first)
            first = False
            self.steps[i] += 1

    def _step_sources(self, sources, sums) -> None:
        """The arena step forming pending gradient sources as it reads the
        gradients, its finishing launch also forming the queued ordered
        sums (ttrl_adam_step_sources)."""
        if len(sources) > MAX_SOURCES:
            settle([t for p in sources[MAX_SOURCES:] for t in p.tensors])
            sources = sources[:MAX_SOURCES]
        if len(sums) > MAX_SUMS:
            self.device.pending_sums.extend(sums[MAX_SUMS:])
            settle_sums(self.device)
            sums = sums[:MAX_SUMS]
        d, _arrays = self._sources_desc(sources, sums)
        self.device.call("ttrl_adam_step_sources", C.byref(d))
        for p in sources:
            p.release()
        self._formed = () if self.store_formed_grads else tuple(sources)

    def materialize_grads(self) -> None:
        """Write the gradients the last step formed without storing them
        (store_formed_grads False) into the parameters' gradient buffers,
        with the step's own formulas and order, so they hold the same bits
        a storing step writes.  Call it after the update and before the next
        launch that reuses the operands (the next update on this device)."""
        formed = self._formed
        if not formed:
            return
        for i in range(0, len(formed), MAX_SOURCES):
            chunk = formed[i:i + MAX_SOURCES]
            arr = (_lib.GradSource * len(chunk))(*[p.source for p in chunk])
            self.device.call("ttrl_grad_sources_materialize", len(chunk), arr)

    def _sources_desc(self, sources, sums):
        """-> (the AdamSourcesDesc of an arena step forming `sources` and the
        ordered `sums`, the ctypes arrays it points to)."""
        a = self.arena
        srcs = (_lib.GradSource * max(1, len(sources)))(*[p.source for p in sources])
        osums = (_lib.OrderedSum * max(1, len(sums)))(*[s for s, _ in sums])
        d = _lib.AdamSourcesDesc(a.data.ptr, a.grad.ptr, self._m_flat.ptr, self._v_flat.ptr, a.numel,
                                 self._counter(len(self.params)).value, self.lr, self.b1, self.b2, self.eps,
                                 self.weight_decay, self.grad_sq.ptr, 0, len(sources), srcs, len(sums), osums,
                                 int(self.store_formed_grads))
        return d, (srcs, osums)

    # -- deferred steps ------------------------------------------------------

    def _hyper(self) -> tuple:
        return (C.c_float(self.lr), C.c_float(self.b1), C.c_float(self.b2), C.c_float(self.eps),
                C.c_float(self.weight_decay))

    def _arena_ready(self, who: str) -> None:
        """The arena launch's preconditions; moves every gradient into its slot."""
        if self.arena is None:
            raise ValueError(f"Adam.{who}: the parameters must be exactly one ParamArena's")
        missing = [i for i, p in enumerate(self.params) if p.grad is None]
        if missing:
            raise RuntimeError(f"Adam.{who}: parameters {missing} hold no gradient for this step")
        if any(st != self._arena_t for st in self.steps):
            raise RuntimeError(f"Adam.{who}: the parameters' update counts differ; use step()")
        settle(self.params)
        for p in self.params:
            if p.grad is not p._grad_slot:
                p._grad_slot.copy_from(p.grad)
                p.grad = p._grad_slot
                p._grad_owned = True

    def step_clipped(self, max_norm: float, sq_out, norm_out, end=None) -> None:
        """clip_grad_norm over the arena's gradient, then step(), with one
        read of the gradient (ttrl_adam_step_clipped): the same parameters,
        moments and clipped gradient as ttrl_clip_grad_norm followed by the
        step.  sq_out and norm_out (device float pointers, nullable) receive
        sum(g^2) and the norm before clipping.  end = (counter, metrics, n,
        ring, slots) also ends a replayed learner step as ttrl_step_end does,
        in the step's finishing launch (ttrl_adam_step_clipped_end)."""
        if not max_norm > 0:
            raise ValueError(f"clip_grad_norm: max_norm must be > 0, got {max_norm}")
        self._arena_ready("step_clipped")
        settle_sums(self.device)
        a = self.arena
        args = (a.data.vp, a.grad.vp, self._m_flat.vp, self._v_flat.vp, C.c_long(a.numel),
                self._counter(len(self.params)), *self._hyper(), self.grad_sq.vp, 0, C.c_float(max_norm), sq_out,
                norm_out)
        if end is None:
            self.device.call("ttrl_adam_step_clipped", *args)
        else:
            counter, metrics, n, ring, slots = end
            self.device.call("ttrl_adam_step_clipped_end", *args, counter, metrics, int(n), ring, int(slots))
        self._finished()

    def step_deferred(self, slot: int) -> None:
        """The arena's update with its finish left to `finish_steps`: the
        update count is read, not stored, and the partial sums of g^2 wait in
        the device context's partial slot `slot` (0-7)."""
        self._arena_ready("step_deferred")
        a = self.arena
        self.device.call("ttrl_adam_step_deferred", a.data.vp, a.grad.vp, self._m_flat.vp, self._v_flat.vp,
                         C.c_long(a.numel), self._counter(len(self.params)), *self._hyper(), int(slot))

    def deferred_range(self, slot: int) -> "_lib.AdamRange":
        """This arena's update as one range of `adam_multi`."""
        self._arena_ready("deferred_range")
        a = self.arena
        return _lib.AdamRange(a.data.ptr, a.grad.ptr, self._m_flat.ptr, self._v_flat.ptr, a.numel,
                              self._counter(len(self.params)).value, self.lr, self.b1, self.b2, self.eps,
                              self.weight_decay, int(slot))

    def fused_range(self, slot: int) -> "_lib.AdamRange":
        """This arena's update as a range that a fused update stage applies
        while it forms the gradients (it writes each gradient into the
        arena's slot, then steps that element); finished by `finish_steps`
        with the stage's partial count."""
        if self.arena is None:
            raise ValueError("Adam.fused_range: the parameters must be exactly one ParamArena's")
        if any(st != self._arena_t for st in self.steps):
            raise RuntimeError("Adam.fused_range: the parameters' update counts differ; use step()")
        a = self.arena
        return _lib.AdamRange(a.data.ptr, a.grad.ptr, self._m_flat.ptr, self._v_flat.ptr, a.numel,
                              self._counter(len(self.params)).value, self.lr, self.b1, self.b2, self.eps,
                              self.weight_decay, int(slot))

    def _finish_desc(self, slot: int, parts: int = 0) -> "_lib.AdamFinish":
        return _lib.AdamFinish(int(slot), self.arena.numel, self._counter(len(self.params)).value,
                               self.grad_sq.ptr, 0, int(parts))

    def _finished(self) -> None:
        """Host counters after a finished step (a capture advances them at replay)."""
        if not self.device.capturing:
            self.t += 1
            self._arena_t += 1
            self.steps = [st + 1 for st in self.steps]

    def arena_grads(self) -> DeviceArray:
        """The arena's flat gradient, after moving every parameter's gradient
        into its slot there (what a global-norm clip reads before the step)."""
        if self.arena is None:
            raise ValueError("Adam.arena_grads: the parameters are not one ParamArena's")
        for p in self.params:
            if p.grad is None:
                raise RuntimeError("Adam.arena_grads: every parameter needs this step's gradient")
        settle(self.params)
        for p in self.params:
            if p.grad is not p._grad_slot:
                p._grad_slot.copy_from(p.grad)
                p.grad = p._grad_slot
                p._grad_owned = True
        return self.arena.grad

    def _step_one(self, i, p, g, args, accumulate):
        dev = self.device
        pd, m, v = p.data, self.m[i], self.v[i]
        staged = [_aligned_copy(x) if (x.ptr % 16) else x for x in (pd, m, v)]
        dev.call("ttrl_adam_step", staged[0].vp, g.vp, staged[1].vp, staged[2].vp, C.c_long(pd.numel),
                 self._counter(i), *args, self.grad_sq.vp, int(accumulate))
        for orig, st in zip((pd, m, v), staged):
            if st is not orig:
                orig.copy_from(st)

    def _replayed(self, have_grads=None) -> None:
        """Host bookkeeping after a graph replay that ran one step."""
        self.t += 1
        self._arena_t += 1
        self.steps = [s + 1 for s in self.steps]

    # -- checkpointing -----------------------------------------------------

    def state_dict(self) -> dict:
        return {
            "t": self.t,
            "steps": list(self.steps),
            "lr": self.lr,
            "betas": (self.b1, self.b2),
            "eps": self.eps,
            "weight_decay": self.weight_decay,
            # Canonical m and v in float64: S * scale / scale then returns the
            # stored float32 S exactly, so a restore resumes bit for bit.
            "m": [m.numpy().astype(np.float64) * self._m_scale for m in self.m],
            "v": [v.numpy().astype(np.float64) * self._v_scale for v in self.v],
        }

    def load_state_dict(self, state: dict, device=None) -> None:
        if len(state["m"]) != len(self.m) or len(state["v"]) != len(self.v):
            raise ValueError(
                f"Adam.load_state_dict: checkpoint has {len(state['m'])} m and {len(state['v'])} v buffers, "
                f"expected {len(self.m)} of each for this optimizer's parameter list."
            )
        for key, buffers in (("m", self.m), ("v", self.v)):
            for i, (arr, buf) in enumerate(zip(state[key], buffers)):
                got = tuple(np.asarray(arr).shape)
                if got != tuple(buf.shape):
                    raise ValueError(
                        f"Adam.load_state_dict: {key}[{i}] has shape {got}, which does not match its "
                        f"parameter's shape {tuple(buf.shape)}."
                    )
        t = int(state["t"])
        steps = [int(s) for s in state.get("steps", [t] * len(self.params))]
        self.lr = float(state.get("lr", self.lr))
        self.b1, self.b2 = (float(x) for x in state.get("betas", (self.b1, self.b2)))
        self.eps = float(state.get("eps", self.eps))
        self.weight_decay = float(state.get("weight_decay", self.weight_decay))
        for arr, buf in zip(state["m"], self.m):
            buf.upload(np.asarray(arr, np.float64) / self._m_scale)
        for arr, buf in zip(state["v"], self.v):
            buf.upload(np.asarray(arr, np.float64) / self._v_scale)
        self.t = t
        self.steps = steps
        self._arena_t = steps[0] if steps and all(s == steps[0] for s in steps) else -1
        self._counters.upload(np.asarray(self.steps + [max(self._arena_t, 0)], np.int32))


def _aligned_copy(x: DeviceArray) -> DeviceArray:
    n = x.numel
    padded = DeviceArray(x.dev, (((n + 3) // 4) * 4,))
    padded.fill(0.0)
    padded.view(0, x.shape).copy_from(x)
    out = padded.view(0, x.shape)
    return out


def adam_multi(device, ranges, polyak=None) -> None:
    """One launch: the deferred updates `ranges` ([(optimizer, slot)], at
    most four) and, with polyak=(dst, src, tau) (DeviceArrays of one
    length), dst = (1 - tau) dst + tau src (ttrl/algos/sac/targets.py:45-52)."""
    descs = [opt.deferred_range(slot) for opt, slot in ranges]
    arr = (_lib.AdamRange * max(1, len(descs)))(*descs)
    if polyak is not None:
        dst, src, tau = polyak
        if dst.numel != src.numel:
            raise ValueError(f"adam_multi: Polyak buffers differ in length ({dst.numel} vs {src.numel})")
        pd, ps, pn = dst.vp, src.vp, dst.numel
    else:
        pd, ps, pn, tau = None, None, 0, 0.0
    device.call("ttrl_adam_multi", len(descs), arr, pd, ps, C.c_long(pn), C.c_float(tau))


def finish_steps(device, steps) -> None:
    """Finishes deferred steps ([(optimizer, slot)] or [(optimizer, slot,
    parts)], parts the number of partial sums a fused stage left in the
    slot) in one launch: each optimizer's sum(g^2) into its `grad_sq` and its
    update count stored."""
    descs = [step[0]._finish_desc(*step[1:]) for step in steps]
    arr = (_lib.AdamFinish * max(1, len(descs)))(*descs)
    device.call("ttrl_adam_finish_slots", len(descs), arr)
    for step in steps:
        step[0]._finished()
