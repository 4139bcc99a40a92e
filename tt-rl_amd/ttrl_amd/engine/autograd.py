"""Reverse-mode autograd tape over device arrays.

Same contract as the reference tape (ttrl/engine/autograd.py:30-271): a
`Tensor` node holds `data`, `requires_grad`, `grad`, a `_backward(grad)`
closure and its `_parents`; `backward()` seeds 1.0 on a scalar, runs every
closure once, each after all of its node's gradient has accumulated (in
fp32), and releases the tape afterwards even on failure.  It refuses a
non-scalar root, a second pass and a root with no tape, with the
reference's messages (its tests match them).

Two MI355X-side additions, invisible to callers:
* a gradient may be written by a kernel straight into its final buffer:
  `_grad_target()` hands out (buffer, beta) so a fused backward accumulates
  in its epilogue instead of through a separate add, and parameters built
  inside a `ParamArena` own a fixed gradient slot;
* the seed is flagged as exactly 1.0, so a fused loss backward skips the
  multiply by its upstream gradient.
"""

from __future__ import annotations

import numpy as np

from ttrl_amd.engine.tensor import DeviceArray, ParamArena, to_device, to_host

__all__ = ["Tensor", "backward", "no_grad", "is_grad_enabled"]

_GRAD_ENABLED = True


def is_grad_enabled() -> bool:
    return _GRAD_ENABLED


class no_grad:
    """Ops built inside record no tape (ttrl/engine/autograd.py:30-44)."""

    def __enter__(self):
        global _GRAD_ENABLED
        self._prev = _GRAD_ENABLED
        _GRAD_ENABLED = False
        return self

    def __exit__(self, *exc):
        global _GRAD_ENABLED
        _GRAD_ENABLED = self._prev
        return False


#: Ops whose output is a ReLU output (their backward applies relu_bw).
# Fused loss nodes whose backward, given a gradient marked `unit`, reads only
# the mark (dQ etc. are already scaled for a unit seed); backward() seeds
# them without filling the seed buffer.
UNIT_SEED_OPS = frozenset({"dqn_td_loss", "sac_critic_loss", "sac_actor_loss", "sac_alpha_loss", "ppo_objective"})
RELU_OPS = frozenset({"linear_relu", "conv2d_relu"})


def relu_mask(t: "Tensor"):
    """The array whose positive entries gate t's gradient when t is a ReLU
    output (possibly through reshapes, which share its buffer), else None."""
    s = t
    while s._op == "reshape" and s._parents:
        s = s._parents[0]
    return t.data if s._op in RELU_OPS else None


def _no_backward(grad):
    return None


class Tensor:
    """A node in the autograd graph, backed by a `DeviceArray`."""

    __slots__ = ("data", "requires_grad", "grad", "_backward", "_parents", "_op", "_backward_done",
                 "_grad_slot", "_grad_owned", "_arena", "_grad_masked", "_pending", "__weakref__")

    def __init__(self, data, requires_grad: bool = False, _parents=(), _op: str = ""):
        self.data = data
        self.requires_grad = requires_grad
        self.grad = None
        self._backward = _no_backward
        self._parents = tuple(_parents)
        self._op = _op
        self._backward_done = False
        self._grad_slot = None
        self._grad_owned = False
        self._arena = None
        # True while every contribution to `grad` was already multiplied by
        # [data > 0]: a consumer applied this node's ReLU backward in its own
        # epilogue, so this node's backward must not apply it again (it would
        # be harmless, but it costs a pass).
        self._grad_masked = False
        # A gradient source (engine.pending) that will write `grad`: set
        # while an earlier launch left this gradient unreduced.
        self._pending = None

    # -- construction ------------------------------------------------------

    @staticmethod
    def from_numpy(array, device, *, requires_grad=False, dtype=np.float32, layout=None) -> "Tensor":
        arr = np.asarray(array)
        t = Tensor(to_device(arr, device, dtype), requires_grad)
        arena = ParamArena.current()
        if requires_grad and arena is not None and t.data.dtype == np.float32:
            arena.register(t)
        return t

    def numpy(self) -> np.ndarray:
        return to_host(self.data)

    # -- introspection -----------------------------------------------------

    @property
    def shape(self):
        return tuple(self.data.shape)

    @property
    def device(self):
        return self.data.dev

    @property
    def dtype(self):
        return self.data.dtype

    def __repr__(self):
        return f"Tensor(shape={self.shape}, op={self._op or 'leaf'}, grad={self.requires_grad})"

    # -- gradient plumbing -------------------------------------------------

    def _accumulate(self, grad: DeviceArray, masked: bool = False):
        """grad += g (ttrl/engine/autograd.py:106-114); `masked` says g was
        already multiplied by this node's ReLU gate."""
        from ttrl_amd.engine.ops import _kernels as K

        self._grad_masked = masked and (self.grad is None or self._grad_masked)
        if self._pending is not None:
            from ttrl_amd.engine.pending import settle
            settle([self])
        if grad.shape != self.shape:
            grad = grad.reshape(self.shape)
        if self.grad is None:
            if self._grad_slot is not None:
                self._grad_slot.copy_from(grad)
                self.grad = self._grad_slot
                self._grad_owned = True
            else:
                self.grad = grad
                self._grad_owned = False
            return
        if self._grad_owned:
            K.binary_into("add", self.grad, grad, self.grad)
        else:
            out = K.binary("add", self.grad, grad)
            self.grad = out
            self._grad_owned = True

    def _grad_target(self):
        """(buffer, beta) a kernel writes this tensor's gradient into.

        beta is 0.0 for the first contribution (overwrite) and 1.0 after
        (accumulate).  The buffer is exclusively this tensor's.
        """
        if self._pending is not None:
            from ttrl_amd.engine.pending import settle
            settle([self])
        if self.grad is None:
            buf = self._grad_slot if self._grad_slot is not None else DeviceArray(self.device, self.shape)
            self.grad = buf
            self._grad_owned = True
            return buf, 0.0
        if not self._grad_owned:
            own = self._grad_slot if self._grad_slot is not None else DeviceArray(self.device, self.shape)
            own.copy_from(self.grad)
            self.grad = own
            self._grad_owned = True
        return self.grad, 1.0

    def _note_write(self, beta: float, masked: bool):
        """Record a kernel's write into the buffer `_grad_target` handed out
        (beta 0 overwrote, 1 accumulated), `masked` as for `_accumulate`."""
        self._grad_masked = masked and (beta == 0.0 or self._grad_masked)

    def zero_grad(self):
        if self._pending is not None:
            # a source writes all of its gradients together: zeroing one of
            # them drops it as a whole
            self._pending.release()
        self.grad = None
        self._grad_owned = False
        self._grad_masked = False

    def detach(self) -> "Tensor":
        return Tensor(self.data, requires_grad=False)

    def backward(self):
        """Run every recorded backward closure once, from this scalar root.

        Order: a node runs only after every node that consumes it has run
        (all of its gradient contributions have arrived).  Each reachable
        node's count of reachable consumers is taken in one sweep; the walk
        then pops ready nodes from a stack and releases a parent when its
        count reaches zero.  The tape is torn down in a `finally`, so saved
        activations go whether the walk finished or raised."""
        if not self.requires_grad:
            raise RuntimeError(
                "backward() called on a Tensor that requires no gradient; it "
                "carries no tape (a leaf, a detached node, or built inside "
                "no_grad()), so this call would silently produce no parameter "
                "gradients at all."
            )
        if self._backward_done:
            raise RuntimeError(
                "backward() called a second time on the same graph; this tape "
                "does not keep saved activations alive for a second pass "
                "(no retain_graph). Build a fresh forward pass instead."
            )
        numel = int(np.prod(self.shape, dtype=np.int64))
        if numel != 1:
            raise RuntimeError(
                f"backward() called on a non-scalar Tensor with shape {self.shape} "
                f"(numel={numel}); there is no `gradient=` kwarg to seed a "
                "non-scalar backward pass, so reduce to a scalar first."
            )
        order = _consumers_first(self)
        seed = DeviceArray(self.device, self.shape)
        if self._op in UNIT_SEED_OPS:
            seed.unit = True  # the root's backward reads only the flag: no fill launch
        else:
            seed.fill(1.0)
        self.grad = seed
        self._grad_owned = True
        try:
            for node in order:
                if node.grad is None:
                    continue
                if node._backward_done and node is not self:
                    raise RuntimeError(
                        "backward() reached a node whose tape was already "
                        "consumed by a previous backward() call on a graph "
                        "sharing this subgraph; reusing a consumed subgraph "
                        "is not supported (no retain_graph)."
                    )
                node._backward(node.grad)
        finally:
            for node in order:
                # Leaves begin the next step's graph: only op nodes are spent.
                node._backward_done = node._backward_done or bool(node._op)
                node._backward = _no_backward
                node._parents = ()


def _consumers_first(root: Tensor) -> list:
    """Nodes reachable from `root`, each after all of its reachable consumers."""
    pending: dict[int, int] = {}
    frontier, reached = [root], {id(root)}
    while frontier:
        for parent in frontier.pop()._parents:
            key = id(parent)
            pending[key] = pending.get(key, 0) + 1
            if key not in reached:
                reached.add(key)
                frontier.append(parent)
    order, ready = [], [root]
    while ready:
        node = ready.pop()
        order.append(node)
        for parent in node._parents:
            key = id(parent)
            pending[key] -= 1
            if pending[key] == 0:
                ready.append(parent)
    return order


# Python operators -> (op name in ttrl_amd.engine.ops.elementwise, operands swapped)
_OPERATORS = {
    "__add__": ("add", False), "__radd__": ("add", True),
    "__sub__": ("sub", False), "__rsub__": ("sub", True),
    "__mul__": ("mul", False), "__rmul__": ("mul", True),
    "__truediv__": ("div", False),
}


def _operator(op_name: str, swapped: bool):
    def method(self, other):
        from ttrl_amd.engine.ops import elementwise

        fn = getattr(elementwise, op_name)
        return fn(other, self) if swapped else fn(self, other)

    method.__name__ = op_name
    return method


def _negate(self):
    from ttrl_amd.engine.ops.elementwise import mul

    return mul(self, -1.0)


for _dunder, (_op_name, _swapped) in _OPERATORS.items():
    setattr(Tensor, _dunder, _operator(_op_name, _swapped))
Tensor.__neg__ = _negate


def backward(tensor: Tensor) -> None:
    tensor.backward()


def _is_scalar(x) -> bool:
    return not isinstance(x, Tensor) and not hasattr(x, "shape")


def _needs(*tensors) -> bool:
    return _GRAD_ENABLED and any(isinstance(t, Tensor) and t.requires_grad for t in tensors)


def _detached(data) -> Tensor:
    return Tensor(data, requires_grad=False)
