"""The engine's generic op surface (ttrl/engine/ops/__init__.py:32-44) on the
GPU against float64 references: forward values and gradients of add / sub /
mul / div with broadcasting and python-number operands, the unary ops, the
relu-identity selections with their tie and bound rules
(ttrl/engine/ops/select.py:26-63), the reductions, detached max / argmax
(first index on ties), concat / split / reshape, one_hot_device,
gather_onehot, one_hot_gather, apply_done_mask, huber, log_softmax, entropy,
matmul and non_finite_check.  Cases follow the reference's op tests
(tests/engine/test_ops_functional.py, tests/engine/test_ops_broadcast.py).

Every differentiable case builds loss = sum(f(inputs) * w) with a fixed
random w, runs the tape, and compares the forward and every input gradient
with torch float64 autograd on the CPU (or a closed form where the
reference's tie rule differs from torch's).  Tolerance: rel 1e-5 of each
tensor's max |value| (rel 2e-5 for matmul)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

REL = 1e-5


def _rel(got, ref):
    ref = np.asarray(ref, np.float64)
    got = np.asarray(got, np.float64).reshape(ref.shape)
    return float(np.max(np.abs(got - ref)) / max(np.max(np.abs(ref)), 1e-30))


def _t(device, arr, grad=True):
    from ttrl_amd.engine.autograd import Tensor
    return Tensor.from_numpy(np.asarray(arr, np.float32), device, requires_grad=grad)


def _run(device, fn_engine, fn_torch, arrays, rel=REL, seed=0):
    """Forward + gradients of sum(f(x) * w) on the device and in torch float64."""
    from ttrl_amd.engine import ops

    xs = [_t(device, a) for a in arrays]
    y = fn_engine(*xs)
    w = np.random.default_rng(seed).standard_normal(y.shape).astype(np.float32)
    loss = ops.sum_all(ops.mul(y, _t(device, w, grad=False)))
    loss.backward()
    tx = [torch.tensor(np.asarray(a, np.float64), requires_grad=True) for a in arrays]
    ty = fn_torch(*tx)
    (ty * torch.tensor(w.astype(np.float64))).sum().backward()
    assert _rel(y.numpy(), ty.detach().numpy()) < rel
    for i, (x, t) in enumerate(zip(xs, tx)):
        assert x.grad is not None, i
        assert _rel(x.grad.numpy(), t.grad.numpy()) < rel, i
    return xs, y


@pytest.mark.parametrize("name", ["add", "sub", "mul", "div"])
@pytest.mark.parametrize("shapes", [((4, 5), (4, 5)), ((4, 5), (1, 5)), ((4, 5), (4, 1)), ((2, 3, 4), (3, 1)),
                                    ((5,), (3, 5)), ((32, 512), (512,))])
def test_binary_broadcast_forward_and_grads(device, name, shapes):
    from ttrl_amd.engine import ops

    rng = np.random.default_rng(hash((name,) + shapes) % 2**32)
    a = rng.standard_normal(shapes[0])
    b = rng.standard_normal(shapes[1])
    if name == "div":
        b = np.sign(b) * (0.5 + np.abs(b))
    torch_fn = {"add": torch.add, "sub": torch.sub, "mul": torch.mul, "div": torch.div}[name]
    _run(device, getattr(ops, name), torch_fn, [a, b])


@pytest.mark.parametrize("name,side", [("add", "rhs"), ("add", "lhs"), ("sub", "rhs"), ("sub", "lhs"),
                                       ("mul", "rhs"), ("mul", "lhs"), ("div", "rhs")])
def test_python_number_operands(device, name, side):
    from ttrl_amd.engine import ops

    c = 1.75
    a = np.random.default_rng(3).standard_normal((6, 7))
    eng, ref = getattr(ops, name), {"add": torch.add, "sub": torch.sub, "mul": torch.mul, "div": torch.div}[name]
    if side == "rhs":
        _run(device, lambda x: eng(x, c), lambda x: ref(x, c), [a])
    else:
        _run(device, lambda x: eng(c, x), lambda x: ref(torch.full_like(x, c), x), [a])


def test_python_number_on_the_left_of_div_is_refused(device):
    from ttrl_amd.engine import ops
    with pytest.raises(TypeError):
        ops.div(2.0, _t(device, np.ones((2, 2))))


def test_operator_methods(device):
    """Tensor +, -, *, /, unary -, and their reflected forms."""
    a = np.random.default_rng(4).standard_normal((3, 4)) + 3.0
    b = np.random.default_rng(5).standard_normal((3, 4)) + 3.0
    _run(device, lambda x, y: (x + y) * 2.0 - 1.0 / 1.0 + (3.0 - x) / y + (-y) + 2.0 * x + (1.0 + y),
         lambda x, y: (x + y) * 2.0 - 1.0 + (3.0 - x) / y + (-y) + 2.0 * x + (1.0 + y), [a, b])


@pytest.mark.parametrize("name", ["relu", "abs_", "exp", "log", "tanh", "sigmoid", "sqrt", "square", "neg"])
def test_unary_forward_and_grads(device, name):
    from ttrl_amd.engine import ops

    x = np.random.default_rng(6).standard_normal((9, 33)) * 2.0
    if name in ("log", "sqrt"):
        x = np.abs(x) + 0.1
    if name in ("relu", "abs_"):
        x = np.where(np.abs(x) < 1e-3, 0.5, x)  # away from the kink: ties are checked separately
    ref = {"relu": torch.relu, "abs_": torch.abs, "exp": torch.exp, "log": torch.log, "tanh": torch.tanh,
           "sigmoid": torch.sigmoid, "sqrt": torch.sqrt, "square": torch.square, "neg": torch.neg}[name]
    _run(device, getattr(ops, name), ref, [x])


def test_relu_and_abs_gradient_at_zero_is_zero(device):
    from ttrl_amd.engine import ops

    for fn in (ops.relu, ops.abs_):
        x = _t(device, np.array([[-1.0, 0.0, 2.0]]))
        ops.sum_all(fn(x)).backward()
        got = x.grad.numpy().reshape(-1)
        assert got[1] == 0.0, fn.__name__


def test_minimum_maximum_forward_grads_and_ties(device):
    """min(a, b) = a - relu(a - b): on a tie the gradient goes to the first
    operand; max(a, b) = a + relu(b - a): likewise to the first operand."""
    from ttrl_amd.engine import ops

    a = np.array([[1.0, 2.0, 3.0, -1.0, 0.5]])
    b = np.array([[2.0, 2.0, 1.0, -1.0, 0.25]])
    for fn, pick in ((ops.minimum, np.minimum), (ops.maximum, np.maximum)):
        ta, tb = _t(device, a), _t(device, b)
        y = fn(ta, tb)
        ops.sum_all(y).backward()
        assert np.array_equal(y.numpy(), pick(a, b).astype(np.float32))
        to_a = (a == pick(a, b))  # ties count as the first operand's
        assert np.array_equal(ta.grad.numpy(), to_a.astype(np.float32)), fn.__name__
        assert np.array_equal(tb.grad.numpy(), (~to_a).astype(np.float32)), fn.__name__
    # a python-number second operand
    ta = _t(device, a)
    y = ops.minimum(ta, 1.0)
    ops.sum_all(y).backward()
    assert np.array_equal(y.numpy(), np.minimum(a, 1.0).astype(np.float32))
    assert np.array_equal(ta.grad.numpy(), (a <= 1.0).astype(np.float32))


def test_clamp_forward_and_zero_gradient_at_the_bounds(device):
    from ttrl_amd.engine import ops

    x = np.array([[-3.0, -2.0, -1.5, 0.0, 1.0, 2.0, 5.0]])
    tx = _t(device, x)
    y = ops.clamp(tx, -2.0, 2.0)
    ops.sum_all(y).backward()
    assert np.array_equal(y.numpy(), np.clip(x, -2.0, 2.0).astype(np.float32))
    inside = (x > -2.0) & (x < 2.0)
    assert np.array_equal(tx.grad.numpy(), inside.astype(np.float32))


@pytest.mark.parametrize("keepdim", [True, False])
def test_sum_and_mean_along_a_dim(device, keepdim):
    from ttrl_amd.engine import ops

    x = np.random.default_rng(7).standard_normal((4, 6, 5))
    for dim in (0, 1, -1):
        _run(device, lambda t: ops.sum_dim(t, dim, keepdim), lambda t: t.sum(dim=dim, keepdim=keepdim), [x])
        _run(device, lambda t: ops.mean_dim(t, dim, keepdim), lambda t: t.mean(dim=dim, keepdim=keepdim), [x])


def test_sum_all_and_mean_all(device):
    from ttrl_amd.engine import ops

    x = np.random.default_rng(8).standard_normal((32, 7))
    for fn, ref in ((ops.sum_all, torch.sum), (ops.mean_all, torch.mean)):
        tx = _t(device, x)
        y = fn(tx)
        y.backward()
        t = torch.tensor(x, requires_grad=True)
        ref(t).backward()
        assert _rel(y.numpy().reshape(-1), [float(ref(torch.tensor(x)))]) < REL
        assert _rel(tx.grad.numpy(), t.grad.numpy()) < REL


def test_detached_max_and_argmax_first_index_on_ties(device):
    from ttrl_amd.engine import ops

    x = np.array([[1.0, 3.0, 3.0, 0.0], [5.0, 5.0, 5.0, 5.0], [-1.0, -2.0, -0.5, -0.5], [0.0, 0.0, 0.0, 1.0]])
    tx = _t(device, x, grad=True)
    m = ops.max_dim_detached(tx, dim=1)
    a = ops.argmax_dim_detached(tx, dim=1)
    assert not m.requires_grad and not a.requires_grad
    assert np.array_equal(m.numpy().reshape(-1), x.max(1).astype(np.float32))
    assert np.array_equal(a.numpy().reshape(-1), np.argmax(x, 1).astype(np.float32))
    big = np.random.default_rng(9).standard_normal((64, 18)).astype(np.float32)
    big[:, 5] = big.max(1) + 1.0
    big[::3, 11] = big[::3, 5]  # exact ties: the first index wins
    got = ops.argmax_dim_detached(_t(device, big, grad=False), dim=-1).numpy().reshape(-1)
    assert np.array_equal(got, np.argmax(big, 1).astype(np.float32))
    assert np.all(got == 5.0)


def test_concat_split_reshape(device):
    from ttrl_amd.engine import ops

    rng = np.random.default_rng(10)
    s, a = rng.standard_normal((256, 11)), rng.standard_normal((256, 3))
    _run(device, lambda x, y: ops.concat([x, y], dim=-1), lambda x, y: torch.cat([x, y], dim=-1), [s, a])
    u, v = rng.standard_normal((2, 5, 3)), rng.standard_normal((4, 5, 3))
    _run(device, lambda x, y: ops.concat([x, y], dim=0), lambda x, y: torch.cat([x, y], dim=0), [u, v])
    g = rng.standard_normal((16, 1536))

    def eng_split(x):
        p = ops.split(x, (512, 512, 512), dim=-1)
        return ops.add(ops.mul(p[0], 2.0), ops.sub(p[2], p[1]))

    def ref_split(x):
        p = torch.split(x, 512, dim=-1)
        return p[0] * 2.0 + (p[2] - p[1])

    _run(device, eng_split, ref_split, [g])
    h = rng.standard_normal((32, 7, 7, 64))
    _run(device, lambda x: ops.reshape(x, (32, 3136)), lambda x: x.reshape(32, 3136), [h])
    with pytest.raises(ValueError):
        ops.split(_t(device, g), (500, 500), dim=-1)


def test_one_hot_device_and_gathers(device):
    from ttrl_amd.engine import ops
    from ttrl_amd.engine.autograd import Tensor

    rng = np.random.default_rng(11)
    B, A = 32, 6
    idx = rng.integers(0, A, B)
    ti = _t(device, idx.reshape(B, 1).astype(np.float32), grad=False)
    oh = ops.one_hot_device(ti, A)
    want = np.eye(A, dtype=np.float32)[idx]
    assert np.array_equal(oh.numpy(), want)
    q = rng.standard_normal((B, A))
    _run(device, lambda x: ops.gather_onehot(x, Tensor(oh.data)),
         lambda x: (x * torch.tensor(want.astype(np.float64))).sum(-1, keepdim=True), [q])
    for indices in (ti, idx):
        tq = _t(device, q)
        y = ops.one_hot_gather(tq, indices, A)
        ops.sum_all(y).backward()
        assert _rel(y.numpy().reshape(-1), q[np.arange(B), idx]) < REL
        assert np.array_equal(tq.grad.numpy(), want)


def test_apply_done_mask_and_huber(device):
    from ttrl_amd.engine import ops

    rng = np.random.default_rng(12)
    v = rng.standard_normal((32, 1))
    done = (rng.random((32, 1)) < 0.3).astype(np.float64)
    _run(device, lambda x, d: ops.apply_done_mask(x, d), lambda x, d: x * (1.0 - d), [v, done])
    pred = rng.standard_normal((32, 1)) * 2.0
    target = rng.standard_normal((32, 1)) * 2.0
    pred[:3, 0] = (0.5, 0.25, 1.5)
    target[:3, 0] = (-0.5, 1.25, 1.5)  # e = +delta, -delta and 0, exact in float32

    def ref_huber(p, t):
        e = (p - t).abs()
        q = torch.minimum(e, torch.ones_like(e))
        return 0.5 * q * q + (e - q)

    tp, tt = _t(device, pred), _t(device, target)
    y = ops.huber(tp, tt, 1.0)
    ops.sum_all(y).backward()
    assert _rel(y.numpy(), ref_huber(torch.tensor(pred), torch.tensor(target)).numpy()) < REL
    # d huber / d pred = clip(e, -delta, delta), and delta * sign(e) at |e| = delta
    e = pred.astype(np.float32).astype(np.float64) - target.astype(np.float32).astype(np.float64)
    assert _rel(tp.grad.numpy(), np.clip(e, -1.0, 1.0)) < REL
    assert _rel(tt.grad.numpy(), -np.clip(e, -1.0, 1.0)) < REL


def test_log_softmax_and_entropy(device):
    from ttrl_amd.engine import ops

    x = np.random.default_rng(13).standard_normal((256, 18)) * 3.0
    _run(device, lambda t: ops.log_softmax(t, -1), lambda t: torch.log_softmax(t, -1), [x])

    def ref_entropy(t):
        lp = torch.log_softmax(t, -1)
        return -(lp.exp() * lp).sum(-1, keepdim=True)

    _run(device, lambda t: ops.entropy(t, -1), ref_entropy, [x])
    # uniform logits: entropy log A
    u = ops.entropy(_t(device, np.zeros((4, 18)), grad=False), -1).numpy()
    assert _rel(u, np.full((4, 1), np.log(18.0))) < REL


@pytest.mark.parametrize("M,K,N", [(32, 3136, 512), (256, 14, 256), (7, 5, 3)])
def test_matmul_forward_and_grads(device, M, K, N):
    from ttrl_amd.engine import ops

    rng = np.random.default_rng(M * 7 + N)
    _run(device, ops.matmul, torch.matmul, [rng.standard_normal((M, K)), rng.standard_normal((K, N))], rel=2e-5)


def test_non_finite_check(device):
    from ttrl_amd.engine import ops

    x = np.ones((4, 4), np.float32)
    assert ops.non_finite_check(_t(device, x, grad=False)) is False
    for bad in (np.nan, np.inf, -np.inf):
        y = x.copy()
        y[2, 3] = bad
        assert ops.non_finite_check(_t(device, y, grad=False)) is True


def test_no_grad_builds_no_tape(device):
    from ttrl_amd.engine import ops
    from ttrl_amd.engine.autograd import no_grad

    x = _t(device, np.ones((2, 2)))
    with no_grad():
        y = ops.mul(ops.exp(x), 2.0)
    assert not y.requires_grad and y._parents == ()
    with pytest.raises(RuntimeError, match="requires no gradient"):
        ops.sum_all(y).backward()


def test_capture_abort_leaves_the_device_usable(device):
    """A capture whose recording reads to host, or raises, is ended and
    discarded (ttrl/engine/trace.py:39-53, :108-125); eager work and a new
    capture then run normally, and the new graph replays correctly."""
    from ttrl_amd.engine import ops
    from ttrl_amd.engine.trace import TraceCaptureError, capture

    base = np.arange(6, dtype=np.float32).reshape(2, 3)
    x = _t(device, base, grad=False)
    ops.mul(x, 3.0)  # a block of the output's size in the pool's free list
    device.synchronize()

    def reads_to_host():
        ops.mul(x, 2.0).numpy()

    with pytest.raises(TraceCaptureError, match="reads a tensor back to host"):
        capture(device, reads_to_host)

    def raises():
        ops.mul(x, 2.0)
        raise ValueError("refused in the recording")

    with pytest.raises(TraceCaptureError, match="refused in the recording"):
        capture(device, raises)
    assert np.array_equal(ops.add(x, 1.0).numpy(), base + 1.0)
    trace, y = capture(device, lambda: ops.mul(x, 3.0))
    try:
        for _ in range(3):
            trace.replay(blocking=True)
            assert np.array_equal(y.numpy(), base * 3.0)
            assert np.array_equal(ops.sub(x, 1.0).numpy(), base - 1.0)  # eager work between replays
    finally:
        trace.close()


def test_frees_during_capture_leave_the_capture_intact(device):
    """A pinned host block or a released pool can be freed while a graph is
    being captured (a garbage collector finalising an unrelated learner
    does it from anywhere).  Releasing either waits for the stream, which a
    capturing stream cannot do; the runtime holds those releases back until
    the capture ends, so the capture succeeds and its graph replays
    correctly, and both are released afterwards."""
    from ttrl_amd.engine import ops
    from ttrl_amd.engine.trace import capture

    base = np.arange(6, dtype=np.float32).reshape(2, 3)
    x = _t(device, base, grad=False)
    ops.mul(x, 5.0)
    block = device.host_block(4096)
    mapped = device.mapped_block(4096)
    pool = device.create_pool()
    with device.use_pool(pool):
        kept = device.alloc(1024)
    device.synchronize()

    def record():
        y = ops.mul(x, 5.0)
        block.close()
        mapped.close()
        device.release_pool(pool)  # retired: one block still live
        device.free(kept)  # the last live block: the slabs go back after the capture
        return ops.add(y, 1.0)

    trace, z = capture(device, record)
    assert device.pool_stats(pool) == (0, 0)  # released once the capture ended
    try:
        for _ in range(3):
            trace.replay(blocking=True)
            assert np.array_equal(z.numpy(), base * 5.0 + 1.0)
    finally:
        trace.close()
    again = device.host_block(4096)  # the context still hands out pinned memory
    again.close()
