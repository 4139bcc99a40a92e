"""Pins of the oracle's DQN update: against torch float64 autograd of the
reference's composition (one-hot gather, relu-identity Huber, IS weights,
mean; ttrl/algos/dqn/losses.py:77-140) on a reduced Nature-CNN, against
central finite differences, against the closed-form Huber gradient, and
a double-vs-vanilla control (tests/hardware/test_algos_dqn_parity.py:129-139)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.dqn import dqn_update, huber
from oracle.nets import QNet, qnet_forward

SHAPE = (4, 36, 36)  # 36 -> 8 -> 3 -> 1 with the Nature-CNN strides


def _net(seed, n_act=6, hidden=32):
    rng = np.random.default_rng(seed)

    def he(shape, fan):
        bnd = np.sqrt(6 / fan)
        return rng.uniform(-bnd, bnd, shape)

    convs = [(he((8, 4, 8, 8), 256), rng.uniform(-.1, .1, 8), 4, 0),
             (he((16, 8, 4, 4), 128), rng.uniform(-.1, .1, 16), 2, 0),
             (he((16, 16, 3, 3), 144), rng.uniform(-.1, .1, 16), 1, 0)]
    fcs = [(he((16, hidden), 16), rng.uniform(-.1, .1, hidden)), (he((hidden, n_act), hidden), rng.uniform(-.1, .1, n_act))]
    return QNet(convs, fcs)


def _batch(seed, B=5, n_act=6):
    from ttrl_amd.workloads import dqn_batch
    return dqn_batch(seed, batch=B, num_actions=n_act, frame_shape=SHAPE)


def _torch_q(net, frames, params):
    x = torch.tensor(np.asarray(frames, np.float64) * net.scale)
    h = x
    it = iter(params)
    for (_, _, s, p) in net.convs:
        w, b = next(it), next(it)
        h = torch.relu(torch.nn.functional.conv2d(h, w, b, stride=s, padding=p))
    h = h.permute(0, 2, 3, 1).reshape(h.shape[0], -1)  # HWC flatten
    last = len(net.fcs) - 1
    for j in range(len(net.fcs)):
        w, b = next(it), next(it)
        h = h @ w + b
        if j < last:
            h = torch.relu(h)
    return h


def _torch_update(net, target, batch, double=True):
    params = [torch.tensor(a, requires_grad=True) for a in net.flat()]
    tparams = [torch.tensor(a) for a in target.flat()]
    q = _torch_q(net, batch["obs"], params)
    with torch.no_grad():
        qn = _torch_q(net, batch["next_obs"], params)
        qt = _torch_q(target, batch["next_obs"], tparams)
        sel = qn if double else qt
        a_star = sel.argmax(1)
        nv = qt.gather(1, a_star[:, None])[:, 0]
        y = torch.tensor(batch["rewards"], dtype=torch.float64) + torch.tensor(batch["discounts"], dtype=torch.float64) * (
            1 - torch.tensor(batch["dones"], dtype=torch.float64)) * nv
    onehot = torch.nn.functional.one_hot(torch.tensor(batch["actions"]), q.shape[1]).double()
    pred = (q * onehot).sum(1)
    ae = (pred - y).abs()
    quad = ae - torch.relu(ae - 1.0)
    h = quad * quad * 0.5 + (ae - quad) * 1.0
    loss = (h * torch.tensor(batch["is_weights"], dtype=torch.float64)).mean()
    loss.backward()
    return float(loss), [p.grad.numpy() for p in params], a_star.numpy(), y.numpy()


@pytest.mark.parametrize("double", [True, False])
def test_dqn_oracle_matches_torch_autograd(double):
    net, target = _net(0), _net(1)
    batch = _batch(2)
    ref = dqn_update(net, target, batch, double=double)
    loss, grads, a_star, y = _torch_update(net, target, batch, double=double)
    assert ref["loss"] == pytest.approx(loss, rel=1e-12)
    assert np.array_equal(ref["next_actions"], a_star)
    np.testing.assert_allclose(ref["td_target"], y, rtol=1e-12)
    for got, want in zip(ref["grads"], grads):
        np.testing.assert_allclose(got.reshape(want.shape), want, rtol=1e-9, atol=1e-12)


def test_double_and_vanilla_targets_differ():
    net, target = _net(3), _net(4)
    batch = _batch(5, B=16)
    a = dqn_update(net, target, batch, double=True)
    b = dqn_update(net, target, batch, double=False)
    assert not np.allclose(a["td_target"], b["td_target"])


def test_dqn_gradient_finite_differences():
    net, target = _net(6), _net(7)
    batch = _batch(8, B=3)
    ref = dqn_update(net, target, batch)
    flat = net.flat()
    rng = np.random.default_rng(9)
    eps = 1e-6
    for idx in range(len(flat)):
        for _ in range(2):
            pos = tuple(rng.integers(0, d) for d in flat[idx].shape)
            plus = [a.copy() for a in flat]
            minus = [a.copy() for a in flat]
            plus[idx][pos] += eps
            minus[idx][pos] -= eps
            # the target and the selection are constants of the step
            fd = (_loss_fixed(net.with_flat(plus), ref, batch) - _loss_fixed(net.with_flat(minus), ref, batch)) / (2 * eps)
            assert fd == pytest.approx(ref["grads"][idx][pos], rel=1e-5, abs=1e-9)


def _loss_fixed(net, ref, batch):
    q, _ = qnet_forward(net, batch["obs"])
    pred = q[np.arange(q.shape[0]), batch["actions"]]
    return float(np.mean(batch["is_weights"] * huber(pred - ref["td_target"], 1.0)))


def test_huber_gradient_closed_form():
    e = np.array([-3.0, -1.0, -0.3, 0.0, 0.4, 1.0, 2.5])
    et = torch.tensor(e, requires_grad=True)
    ae = et.abs()
    quad = ae - torch.relu(ae - 1.0)
    (quad * quad * 0.5 + (ae - quad)).sum().backward()
    np.testing.assert_allclose(et.grad.numpy(), np.clip(e, -1, 1))
    np.testing.assert_allclose(huber(e, 1.0), np.where(np.abs(e) <= 1, 0.5 * e * e, np.abs(e) - 0.5))


def test_three_chained_updates_match_torch_adam():
    """Threading the oracle's Adam state (S, V, t) through three updates
    equals torch.optim.Adam (eps 1.5e-4) driving the torch reproduction:
    pins dqn_update's adam_state / t path, which steps from a learner's
    saved moments."""
    net, target = _net(10), _net(11)
    lr, eps = 6.25e-5, 1.5e-4
    params = [torch.tensor(a, requires_grad=True) for a in net.flat()]
    opt = torch.optim.Adam(params, lr=lr, betas=(0.9, 0.999), eps=eps)
    state, cur = None, net
    for step in range(1, 4):
        batch = _batch(20 + step)
        ref = dqn_update(cur, target, batch, lr=lr, eps=eps, adam_state=state, t=step)
        opt.zero_grad()
        tnet = net.with_flat([p.detach().numpy().copy() for p in params])
        loss, grads, _, _ = _torch_update(tnet, target, batch)
        assert ref["loss"] == pytest.approx(loss, rel=1e-12)
        for p, g in zip(params, grads):
            p.grad = torch.tensor(g)
        opt.step()
        for got, want in zip(ref["new_params"], params):
            np.testing.assert_allclose(got.reshape(want.shape), want.detach().numpy(), rtol=1e-12, atol=1e-15)
        state = (ref["new_S"], ref["new_V"])
        cur = net.with_flat(ref["new_params"])
