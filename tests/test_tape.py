"""Host-only tests of the autograd tape's walk and refusals and of the
capture abort path, on a stand-in device that only records calls (the
reference tests the same logic host-only, tests/engine/test_autograd_tape.py:51-102,
tests/engine/test_autograd_semantics.py:35-52, and its capture abort
ttrl/engine/trace.py:39-53, :108-125).  No GPU and no kernel: the tape's
closures here only record their visit and hand the gradient on."""

from __future__ import annotations

import pytest


class FakeDevice:
    """alloc/free/call/closed: the part of Device a DeviceArray and the tape use."""

    closed = False

    def __init__(self):
        self.calls = []
        self._next = 4096
        self._capturing = False
        self.ctx = None

    def alloc(self, nbytes):
        self._next += 256 * (1 + nbytes // 256)
        return self._next

    def free(self, ptr):
        pass

    def call(self, name, *args):
        self.calls.append(name)


@pytest.fixture
def dev():
    return FakeDevice()


def _node(dev, shape=(1, 1), parents=(), op="", requires_grad=True):
    from ttrl_amd.engine.autograd import Tensor
    from ttrl_amd.engine.tensor import DeviceArray

    return Tensor(DeviceArray(dev, shape), requires_grad, parents, op)


def _wire(root, order):
    """Each op node records its visit and passes its gradient to every parent."""
    stack, seen = [root], set()
    while stack:
        node = stack.pop()
        if id(node) in seen:
            continue
        seen.add(id(node))
        stack.extend(node._parents)
        if not node._op:
            continue

        def make(n):
            def _backward(grad):
                order.append(n._op)
                for p in n._parents:
                    if p.grad is None:
                        p.grad = grad
            return _backward

        node._backward = make(node)


def test_diamond_visits_consumers_before_producers(dev):
    leaf = _node(dev)
    d = _node(dev, parents=(leaf,), op="d")
    b = _node(dev, parents=(d,), op="b")
    c = _node(dev, parents=(d,), op="c")
    a = _node(dev, parents=(b, c), op="a")
    order = []
    _wire(a, order)
    a.backward()
    assert order[0] == "a" and order[-1] == "d"
    assert set(order) == {"a", "b", "c", "d"} and len(order) == 4
    assert dev.calls == ["ttrl_fill_f32"]  # the seed


def test_each_closure_runs_once_on_a_deep_shared_graph(dev):
    """A ladder where every rung feeds the next two: each node runs once, after both consumers."""
    leaf = _node(dev)
    layer = [_node(dev, parents=(leaf,), op="r0a"), _node(dev, parents=(leaf,), op="r0b")]
    for i in range(1, 40):
        layer = [_node(dev, parents=tuple(layer), op=f"r{i}a"), _node(dev, parents=tuple(layer), op=f"r{i}b")]
    root = _node(dev, parents=tuple(layer), op="root")
    order = []
    _wire(root, order)
    root.backward()
    assert len(order) == len(set(order)) == 81
    pos = {name: i for i, name in enumerate(order)}
    for i in range(1, 40):
        for side in "ab":
            assert pos[f"r{i}{side}"] < pos[f"r{i - 1}a"] and pos[f"r{i}{side}"] < pos[f"r{i - 1}b"]


def test_a_parent_listed_twice_waits_for_both_uses(dev):
    leaf = _node(dev)
    x = _node(dev, parents=(leaf,), op="x")
    sq = _node(dev, parents=(x, x), op="sq")
    order = []
    _wire(sq, order)
    sq.backward()
    assert order == ["sq", "x"]


def test_teardown_spares_leaves(dev):
    leaf = _node(dev)
    mid = _node(dev, parents=(leaf,), op="mid")
    root = _node(dev, parents=(mid,), op="root")
    _wire(root, [])
    root.backward()
    assert mid._backward_done and root._backward_done
    assert leaf._backward_done is False
    assert mid._parents == () and root._parents == ()


def test_second_pass_is_refused(dev):
    leaf = _node(dev)
    root = _node(dev, parents=(leaf,), op="root")
    _wire(root, [])
    root.backward()
    with pytest.raises(RuntimeError, match="second time"):
        root.backward()


def test_non_scalar_root_is_refused_before_any_device_work(dev):
    root = _node(dev, shape=(2, 3), parents=(_node(dev),), op="root")
    _wire(root, [])
    with pytest.raises(RuntimeError, match="non-scalar"):
        root.backward()
    assert dev.calls == []


def test_root_without_tape_is_refused(dev):
    detached = _node(dev, op="mul", requires_grad=False)
    with pytest.raises(RuntimeError, match="requires no gradient"):
        detached.backward()


def test_reused_consumed_subgraph_is_refused(dev):
    a, b = _node(dev), _node(dev)
    shared = _node(dev, parents=(a, b), op="shared")
    loss1 = _node(dev, parents=(shared,), op="loss1")
    loss2 = _node(dev, parents=(shared, shared), op="loss2")
    _wire(loss1, [])
    loss1.backward()
    # loss2 was built before loss1's walk tore `shared` down
    loss2._backward = lambda grad: setattr(shared, "grad", grad)
    with pytest.raises(RuntimeError, match="already consumed"):
        loss2.backward()


def test_tape_is_released_when_a_closure_raises(dev):
    leaf = _node(dev)
    mid = _node(dev, parents=(leaf,), op="mid")
    root = _node(dev, parents=(mid,), op="root")
    _wire(root, [])

    def boom(grad):
        raise ValueError("kernel refused")

    mid._backward = boom
    root._backward = lambda grad: setattr(mid, "grad", grad)
    with pytest.raises(ValueError, match="kernel refused"):
        root.backward()
    assert mid._parents == () and root._parents == ()
    assert mid._backward_done and root._backward_done


class _AbortRecorder:
    def __init__(self):
        self.aborts = 0

    def ttrl_capture_abort(self, ctx):
        self.aborts += 1
        return 0


def test_capture_abort_ends_the_capture_and_names_the_failure(dev, monkeypatch):
    from ttrl_amd import _lib
    from ttrl_amd.engine.trace import TraceCaptureError, capture

    rec = _AbortRecorder()
    monkeypatch.setattr(_lib, "lib", lambda: rec)

    def record():
        dev.call("some_kernel")
        raise ValueError("shape refused inside the recording")

    with pytest.raises(TraceCaptureError, match="shape refused"):
        capture(dev, record)
    assert rec.aborts == 1 and dev._capturing is False
    assert dev.calls == ["ttrl_capture_begin", "some_kernel"]

    def host_read():
        raise RuntimeError("ttrl_d2h: reads to host are not supported during graph capture; read metrics after")

    with pytest.raises(TraceCaptureError, match="reads a tensor back to host"):
        capture(dev, host_read)
    assert rec.aborts == 2 and dev._capturing is False


def test_capture_abort_lets_keyboard_interrupt_through(dev, monkeypatch):
    from ttrl_amd import _lib
    from ttrl_amd.engine.trace import capture

    rec = _AbortRecorder()
    monkeypatch.setattr(_lib, "lib", lambda: rec)

    def record():
        raise KeyboardInterrupt

    with pytest.raises(KeyboardInterrupt):
        capture(dev, record)
    assert rec.aborts == 1 and dev._capturing is False
