"""Host bookkeeping of pending gradients and queued batch sums
(ttrl_amd.engine.pending), without a GPU: registration, de-duplication,
release on zero_grad, and the optimizer dropping an abandoned update's
queued sums (a warm-up pass that runs the body without the step)."""

from __future__ import annotations

import pytest


class _Dev:
    def __init__(self):
        self.pending_sums = []


class _Arr:
    def __init__(self, dev):
        self.dev = dev
        self.shape = (4,)


def _tensors(dev, n):
    from ttrl_amd.engine.autograd import Tensor

    return [Tensor(_Arr(dev), requires_grad=True) for _ in range(n)]


def _source(kind=1):
    from ttrl_amd import _lib

    return _lib.GradSource(kind=kind, rows=4, cols=4)


def test_pending_grad_registers_and_releases():
    from ttrl_amd.engine.pending import PendingGrad, take_sources

    dev = _Dev()
    w, b, other = _tensors(dev, 3)
    p = PendingGrad(_source(), (w, b))
    assert w._pending is p and b._pending is p and other._pending is None
    assert take_sources([w, b, other]) == [p]  # one source, listed once
    with pytest.raises(RuntimeError):
        PendingGrad(_source(), (w,))
    # a source writes its gradients together: zeroing one of them drops it
    # as a whole (an abandoned update's zero_grad zeroes them all)
    w.zero_grad()
    assert w._pending is None and b._pending is None


def test_nothing_pending_is_refused():
    from ttrl_amd.engine.pending import PendingGrad

    with pytest.raises(ValueError):
        PendingGrad(_source(kind=0), _tensors(_Dev(), 1))


def test_zero_grad_drops_queued_sums():
    from ttrl_amd.engine.optim import Optimizer
    from ttrl_amd.engine.pending import add_sums, take_sums

    dev = _Dev()
    params = _tensors(dev, 2)
    add_sums(dev, ["loss", "mean_q"], keep=("terms",))
    assert [s for s, _ in dev.pending_sums] == ["loss", "mean_q"]
    Optimizer(params).zero_grad()
    assert dev.pending_sums == []
    add_sums(dev, ["loss"])
    assert [s for s, _ in take_sums(dev)] == ["loss"] and dev.pending_sums == []
