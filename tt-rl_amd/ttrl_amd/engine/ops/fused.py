"""Fused layer and loss ops: one tape node per layer (GEMM + bias + ReLU in
one kernel, masked-ReLU backward and the bias gradient inside the
weight-gradient GEMM) and one per loss head.

`linear` computes exactly `relu(matmul(x, W) + b)` of
ttrl/engine/layers.py:57-61 and ttrl/engine/ops/unary.py:25-37; its backward
gives the same gradients as the reference's matmul / add / relu_bw chain
(ttrl/engine/ops/matmul.py:71-84, ttrl/engine/ops/broadcast.py:11-30).
"""

from __future__ import annotations

import ctypes as C

import numpy as np

from ttrl_amd import _lib
from ttrl_amd.engine.autograd import Tensor, _detached, _needs, relu_mask
from ttrl_amd.engine.pending import PendingGrad, add_sums
from ttrl_amd.engine.tensor import DeviceArray

__all__ = ["linear", "linear_node", "dqn_td_loss", "dqn_head_td_loss", "dqn_tail_td_loss", "grad_targets"]


def _p(arr) -> int | None:
    return None if arr is None else arr.ptr


def grad_targets(*tensors):
    """(buffer, beta) per tensor that requires grad (None otherwise), with a
    common beta.  A mixed first/accumulated set is brought to beta=1 by
    zero-filling the fresh buffers."""
    out = []
    for t in tensors:
        if t is None or not t.requires_grad:
            out.append(None)
            continue
        out.append(list(t._grad_target()))
    betas = {o[1] for o in out if o is not None}
    if len(betas) > 1:
        for o in out:
            if o is not None and o[1] == 0.0:
                o[0].fill(0.0)
                o[1] = 1.0
    beta = 1.0 if 1.0 in betas else 0.0
    return [None if o is None else o[0] for o in out], beta


def linear(x: Tensor, weight: Tensor, bias: Tensor | None = None, *, relu: bool = False) -> Tensor:
    """y = x @ W + b (+ ReLU) as one MFMA launch; W stored (in, out)."""
    if len(x.shape) != 2 or len(weight.shape) != 2:
        raise ValueError(f"linear: expected (M, K) @ (K, N), got {x.shape} @ {weight.shape}")
    M, K = (int(d) for d in x.shape)
    K2, N = (int(d) for d in weight.shape)
    if K != K2:
        raise ValueError(f"linear: input has {K} features, weight expects {K2}")
    if bias is not None and bias.data.numel != N:
        raise ValueError(f"linear: bias has {bias.data.numel} elements, expected {N}")
    dev = x.device
    y = DeviceArray(dev, (M, N))
    d = _lib.LinearDesc()
    d.M, d.K, d.N, d.groups = M, K, N, 1
    d.x, d.ldx = x.data.ptr, K
    d.W = weight.data.ptr
    d.b = _p(bias.data if bias is not None else None)
    d.y = y.ptr
    d.relu = int(relu)
    dev.call("ttrl_linear_forward", C.byref(d))
    return linear_node(x, weight, bias, y, relu=relu)


def linear_node(x: Tensor, weight: Tensor, bias: Tensor | None, y: DeviceArray, *, relu: bool,
                defer: bool = False) -> Tensor:
    """The tape node of y = x @ W + b (+ReLU), with y computed elsewhere.

    defer=True leaves the weight and bias gradients (dW = x^T dZ, db = the
    column sums of dZ) to the optimizer step that follows, as an
    outer-product source over the batch (engine.pending) whose operands are
    x and dZ; the backward then computes only dX.  It applies when the
    gradients are written fresh and dZ arrives already gated."""
    if not _needs(x, weight, bias):
        return _detached(y)
    M, K = (int(dim) for dim in x.shape)
    N = int(weight.shape[1])
    dev = x.device
    parents = (x, weight) + ((bias,) if bias is not None else ())
    out = Tensor(y, True, parents, "linear_relu" if relu else "linear")
    x_data, w_data = x.data, weight.data

    def _backward(grad):
        (dw, db), beta_w = grad_targets(weight, bias)
        (dx,), beta_x = grad_targets(x)
        gate = relu and not out._grad_masked  # relu_bw still to apply to grad
        xmask = relu_mask(x) if dx is not None else None
        if defer and dw is not None and beta_w == 0.0 and not gate and (bias is None or db is not None):
            src = _lib.GradSource(kind=_lib.GRAD_OUTER, rows=K, cols=N, dw=dw.ptr, db=_p(db), u=x_data.ptr,
                                  v=grad.ptr, batch=M)
            PendingGrad(src, (weight, bias), keep=(x_data, grad))
            dw = db = None
        if dw is None and db is not None:
            # Bias-only gradient: a column sum of dZ.
            from ttrl_amd.engine.ops import _kernels as Kk
            g = Kk.binary("relu_bw", grad, y) if gate else grad
            s = Kk.reduce_dim("sum", g, 0, keepdim=True)
            if beta_w:
                Kk.binary_into("add", db, s.reshape(db.shape), db)
            else:
                db.copy_from(s.reshape(db.shape))
            db_ = None
        else:
            db_ = db
        b = _lib.LinearDesc()
        b.M, b.K, b.N, b.groups = M, K, N, 1
        b.x, b.ldx = x_data.ptr, K
        b.W = w_data.ptr
        b.dy = grad.ptr
        b.ymask = y.ptr if gate else None
        b.dxmask = xmask.ptr if xmask is not None else None
        b.dW = _p(dw)
        b.db = _p(db_) if dw is not None else None
        b.dx = _p(dx)
        b.lddx = K
        b.beta_w, b.beta_x = beta_w, beta_x
        if dw is not None or dx is not None:
            dev.call("ttrl_linear_backward", C.byref(b))
        if dx is not None:
            x._note_write(beta_x, xmask is not None)

    out._backward = _backward
    return out


def dqn_td_loss(q: Tensor, q_next_select: Tensor, q_next_value: Tensor, actions_onehot: Tensor,
                rewards: Tensor, dones: Tensor, discounts: Tensor, is_weights: Tensor | None,
                delta: float, out: dict | None = None):
    """The DQN update head as one kernel (ttrl/algos/dqn/losses.py:96-129).

    -> (loss, metrics) where loss is a (1, 1) tape node differentiable in `q`
    and metrics holds detached `mean_q`, `td_abs` (B, 1), `td_target` (B, 1)
    and `next_actions` (B, 1, float indices).  `out` may supply the arrays
    `loss`, `mean_q` and `td_abs` are written to (views of one packed metrics
    block, read back with one copy).
    """
    B, A = (int(d) for d in q.shape)
    for name, t, shape in (("q_next_select", q_next_select, (B, A)), ("q_next_value", q_next_value, (B, A)),
                           ("actions_onehot", actions_onehot, (B, A))):
        if tuple(t.shape) != shape:
            raise ValueError(f"dqn_td_loss: {name} has shape {t.shape}, expected {shape}")
    for name, t in (("rewards", rewards), ("dones", dones), ("discounts", discounts), ("is_weights", is_weights)):
        if t is not None and t.data.numel != B:
            raise ValueError(f"dqn_td_loss: {name} has {t.data.numel} elements, expected {B}")
    if not delta > 0.0:
        raise ValueError(f"dqn_td_loss: huber delta must be > 0, got {delta}")
    dev = q.device
    loss, mean_q, td_abs, td_target, next_act, dq = _dqn_outputs(dev, B, A, out)
    dev.call("ttrl_dqn_loss", B, A, q.data.vp, q_next_select.data.vp, q_next_value.data.vp,
             actions_onehot.data.vp, rewards.data.vp, dones.data.vp, discounts.data.vp,
             None if is_weights is None else is_weights.data.vp, C.c_float(delta), loss.vp, mean_q.vp,
             td_abs.vp, dq.vp, next_act.vp, td_target.vp)
    return _dqn_loss_node(q, loss, mean_q, td_abs, td_target, next_act, dq)


def _dqn_outputs(dev, B: int, A: int, out: dict | None = None):
    """loss, mean_q, td_abs (caller-supplied when `out` names them),
    td_target, next_actions, dq."""
    out = out or {}

    def given(name, shape):
        a = out.get(name)
        if a is None:
            return DeviceArray(dev, shape)
        if a.numel != int(np.prod(shape)) or a.dtype != np.float32:
            raise ValueError(f"DQN loss: out[{name!r}] must hold {int(np.prod(shape))} float32 values")
        return a.reshape(shape)

    return (given("loss", (1, 1)), given("mean_q", (1, 1)), given("td_abs", (B, 1)), DeviceArray(dev, (B, 1)),
            DeviceArray(dev, (B, 1)), DeviceArray(dev, (B, A)))


def _dqn_loss_node(q: Tensor, loss, mean_q, td_abs, td_target, next_act, dq):
    """The loss tape node over q, its dL/dq already computed for a unit seed."""
    metrics = {
        "mean_q": Tensor(mean_q), "td_abs": Tensor(td_abs), "td_target": Tensor(td_target),
        "next_actions": Tensor(next_act),
    }
    if not _needs(q):
        return _detached(loss), metrics
    out = Tensor(loss, True, (q,), "dqn_td_loss")

    def _backward(grad):
        if not q.requires_grad:
            return
        if grad.unit:
            q._accumulate(dq)
        else:
            from ttrl_amd.engine.ops import _kernels as Kk
            q._accumulate(Kk.binary("mul", dq, grad.reshape((1, 1))))

    out._backward = _backward
    return out, metrics


def dqn_head_td_loss(features, heads, actions_onehot: Tensor, rewards: Tensor, dones: Tensor, discounts: Tensor,
                     is_weights: Tensor | None, delta: float, out: dict | None = None):
    """The Q head's last linear layer over 2 or 3 feature sets and the DQN
    loss in one launch (ttrl_dqn_head): features[0] = online(s) (taped),
    features[1] = online(s') selecting a* (double) or target(s'),
    features[-1] = target(s') valuing it; heads[g] the matching Linear.
    -> (loss, metrics, q_arrays) with the same loss node and metrics as
    dqn_td_loss on the three Q tensors; q of group 0 is a linear tape node,
    so the backward is the layer's usual weight / input gradient."""
    G = len(features)
    if G not in (2, 3) or len(heads) != G:
        raise ValueError(f"dqn_head_td_loss: 2 or 3 feature sets and heads, got {G} and {len(heads)}")
    B, K = (int(d) for d in features[0].shape)
    A = int(heads[0].out_features)
    for f, h in zip(features, heads):
        if tuple(f.shape) != (B, K) or int(h.in_features) != K or int(h.out_features) != A:
            raise ValueError("dqn_head_td_loss: feature sets and heads must share (B, K) and (K, A)")
    if tuple(actions_onehot.shape) != (B, A):
        raise ValueError(f"dqn_head_td_loss: actions_onehot has shape {actions_onehot.shape}, expected {(B, A)}")
    for name, t in (("rewards", rewards), ("dones", dones), ("discounts", discounts), ("is_weights", is_weights)):
        if t is not None and t.data.numel != B:
            raise ValueError(f"dqn_head_td_loss: {name} has {t.data.numel} elements, expected {B}")
    if not delta > 0.0:
        raise ValueError(f"dqn_head_td_loss: huber delta must be > 0, got {delta}")
    dev = features[0].device
    weights = [h.effective_weight() for h in heads]
    qs = [DeviceArray(dev, (B, A)) for _ in range(G)]
    loss, mean_q, td_abs, td_target, next_act, dq = _dqn_outputs(dev, B, A, out)
    dev.call("ttrl_dqn_head", B, K, A, G, _lib.ptrs(f.data.ptr for f in features), _lib.ptrs(w.data.ptr for w in weights),
             _lib.ptrs(None if h.bias is None else h.bias.data.ptr for h in heads), _lib.ptrs(q.ptr for q in qs),
             actions_onehot.data.vp, rewards.data.vp, dones.data.vp, discounts.data.vp,
             None if is_weights is None else is_weights.data.vp, C.c_float(delta), loss.vp, mean_q.vp, td_abs.vp,
             dq.vp, next_act.vp, td_target.vp)
    q0 = linear_node(features[0], weights[0], heads[0].bias, qs[0], relu=False)
    out, metrics = _dqn_loss_node(q0, loss, mean_q, td_abs, td_target, next_act, dq)
    return out, metrics, qs


def dqn_tail_td_loss(features, fc1s, fc2s, actions_onehot: Tensor, rewards: Tensor, dones: Tensor,
                     discounts: Tensor, is_weights: Tensor | None, delta: float, out: dict | None = None,
                     defer: bool = False):
    """A Q network's last two layers (Linear -> ReLU -> Linear) over 2 or 3
    feature sets, the DQN loss and the second layer's backward, as one GEMM
    and one kernel (ttrl_dqn_tail): features[0] = online(s) (taped),
    features[1] selects a*, features[-1] values it; fc1s[g] / fc2s[g] the
    matching layers.

    -> (loss, metrics, hs, qs): the loss node and metrics of dqn_td_loss, the
    first layer's outputs and the Q values of every set.  The second layer's
    weight and bias gradients are produced with the loss (they depend on the
    loss alone), so they are written into those parameters' gradients here;
    the loss node's backward hands the first layer's ReLU node its already
    gated gradient.  The loss must be the root of the backward pass.

    defer=True leaves to the update's optimizer step what needs the whole
    batch (engine.pending): the second layer's gradients become an
    outer-product gradient source over h[0] and dq, and the loss and mean Q
    ordered sums of the per-sample terms, so the kernel has no
    cross-workgroup phase.  An optimizer step (or pending.settle and
    settle_sums) must follow before they are read."""
    G = len(features)
    if G not in (2, 3) or len(fc1s) != G or len(fc2s) != G:
        raise ValueError(f"dqn_tail_td_loss: 2 or 3 feature sets and layer pairs, got {G}")
    B, K = (int(d) for d in features[0].shape)
    F, A = int(fc1s[0].out_features), int(fc2s[0].out_features)
    for x, l1, l2 in zip(features, fc1s, fc2s):
        if tuple(x.shape) != (B, K) or (int(l1.in_features), int(l1.out_features)) != (K, F) or \
                (int(l2.in_features), int(l2.out_features)) != (F, A):
            raise ValueError("dqn_tail_td_loss: feature sets and layers must share their shapes")
    if tuple(actions_onehot.shape) != (B, A):
        raise ValueError(f"dqn_tail_td_loss: actions_onehot has shape {actions_onehot.shape}, expected {(B, A)}")
    for name, t in (("rewards", rewards), ("dones", dones), ("discounts", discounts), ("is_weights", is_weights)):
        if t is not None and t.data.numel != B:
            raise ValueError(f"dqn_tail_td_loss: {name} has {t.data.numel} elements, expected {B}")
    if not delta > 0.0:
        raise ValueError(f"dqn_tail_td_loss: huber delta must be > 0, got {delta}")
    head = fc2s[0]
    if head.effective_weight() is not head.weight:
        raise ValueError("dqn_tail_td_loss: the second layer's weight must be its parameter (no scale)")
    dev = features[0].device
    w1 = [l.effective_weight() for l in fc1s]
    hs = [DeviceArray(dev, (B, F)) for _ in range(G)]
    qs = [DeviceArray(dev, (B, A)) for _ in range(G)]
    loss, mean_q, td_abs, td_target, next_act, dq = _dqn_outputs(dev, B, A, out)
    dh = DeviceArray(dev, (B, F))
    (dw2, db2), beta_w = grad_targets(head.weight, head.bias)
    if dw2 is None:
        raise ValueError("dqn_tail_td_loss: the second layer's weight must require a gradient")
    d = _lib.DqnTailDesc()
    d.B, d.K, d.F, d.A, d.groups = B, K, F, A, G
    for g in range(G):
        d.x[g] = features[g].data.ptr
        d.W1[g] = w1[g].data.ptr
        d.b1[g] = _p(None if fc1s[g].bias is None else fc1s[g].bias.data)
        d.h[g] = hs[g].ptr
        d.W2[g] = fc2s[g].weight.data.ptr
        d.b2[g] = _p(None if fc2s[g].bias is None else fc2s[g].bias.data)
        d.q[g] = qs[g].ptr
    d.actions_onehot = actions_onehot.data.ptr
    d.rewards, d.dones, d.discounts = rewards.data.ptr, dones.data.ptr, discounts.data.ptr
    d.is_weights = _p(None if is_weights is None else is_weights.data)
    d.delta = float(delta)
    d.loss, d.mean_q, d.td_abs, d.dq = loss.ptr, mean_q.ptr, td_abs.ptr, dq.ptr
    d.next_actions, d.td_target = next_act.ptr, td_target.ptr
    d.dh, d.dW2, d.db2, d.beta_w = dh.ptr, dw2.ptr, _p(db2), beta_w
    deferred = defer and beta_w == 0.0
    if deferred:
        terms = DeviceArray(dev, (B, 2))
        d.dW2, d.db2, d.loss_terms = None, None, terms.ptr
    dev.call("ttrl_dqn_tail", C.byref(d))
    if deferred:
        src = _lib.GradSource(kind=_lib.GRAD_OUTER, rows=F, cols=A, dw=dw2.ptr, db=_p(db2), u=hs[0].ptr, v=dq.ptr,
                              batch=B)
        PendingGrad(src, (head.weight, head.bias if db2 is not None else None), keep=(hs[0], dq))
        inv_b = float(np.float32(1.0) / np.float32(B))
        sums = [_lib.OrderedSum(terms.ptr, B, 2, inv_b, loss.ptr)]
        if mean_q is not None:
            sums.append(_lib.OrderedSum(terms.ptr + 4, B, 2, inv_b, mean_q.ptr))
        add_sums(dev, sums, keep=(terms,))
    h0 = linear_node(features[0], w1[0], fc1s[0].bias, hs[0], relu=True, defer=deferred)
    metrics = {"mean_q": Tensor(mean_q), "td_abs": Tensor(td_abs), "td_target": Tensor(td_target),
               "next_actions": Tensor(next_act)}
    if not _needs(h0):
        return _detached(loss), metrics, hs, qs
    node = Tensor(loss, True, (h0,), "dqn_td_loss")

    def _backward(grad):
        if not grad.unit:
            raise RuntimeError("dqn_tail_td_loss: the fused loss produces the head's gradients for a unit seed; "
                               "call backward() on the loss itself")
        h0._accumulate(dh, masked=True)

    node._backward = _backward
    return node, metrics, hs, qs
