"""The PPO update oracle (oracle/ppo.py: minibatch_indices, ppo_update) pinned
on the CPU: the shuffle against the reference's rule stated directly
(ttrl/buffers/rollout.py:239-282), and the whole update against an
independent torch float64 reproduction -- autograd through a small
Nature-style tower, the objective composed from torch ops as
ttrl/algos/ppo/loss.py:42-83 writes it, the global-norm clip of
ttrl/algos/grads.py:13-43, and torch.optim.Adam (textbook Adam, which the
reference's fused form equals, ttrl/engine/optim/scalars.py:13-27)."""

from __future__ import annotations

import numpy as np
import pytest


def test_minibatch_indices_follow_the_reference_rule():
    from oracle.ppo import minibatch_indices

    valid = np.ones((5, 4), np.float32)
    valid[1, 2] = 0.0
    valid[3, 0] = 0.0
    got = minibatch_indices(valid, 6, 2, np.random.default_rng(3))
    keep = np.flatnonzero(valid.reshape(-1) > 0)
    rng = np.random.default_rng(3)
    want = []
    for _ in range(2):
        perm = rng.permutation(keep.size)
        want += [keep[perm[s:s + 6]] for s in range(0, (keep.size // 6) * 6, 6)]
    assert len(got) == 2 * (18 // 6)
    for g, w in zip(got, want):
        assert np.array_equal(g, w)
    flat = np.concatenate(got)
    assert 6 not in flat and 12 not in flat  # padding slots never drawn
    with pytest.raises(ValueError):
        minibatch_indices(np.ones((2, 2)), 5, 1, np.random.default_rng(0))


def _small_net(rng, A):
    from oracle.nets import QNet

    def u(shape, fan):
        b = np.sqrt(6.0 / fan)
        return rng.uniform(-b, b, shape)

    convs = [(u((8, 4, 4, 4), 64), u((8,), 64), 2, 0), (u((8, 8, 3, 3), 72), u((8,), 72), 1, 0)]
    fcs = [(u((72, 16), 72), u((16,), 72)), (u((16, A + 1), 16), u((A + 1,), 16))]
    return QNet(convs, fcs, 1.0 / 255.0)


def _torch_update(net, rollout, idx_list, adv_n, ret, cfg):
    import torch

    torch.set_default_dtype(torch.float64)
    params = [torch.tensor(p, requires_grad=True) for p in net.flat()]
    opt = torch.optim.Adam(params, lr=cfg["lr"], eps=cfg["adam_eps"])
    frames = np.asarray(rollout["obs"]).reshape((-1, 4, 12, 12))
    actions = np.asarray(rollout["actions"]).reshape(-1)
    old_logp = np.asarray(rollout["logp"], np.float64).reshape(-1)
    old_v = np.asarray(rollout["values"], np.float64).reshape(-1)
    steps = []
    for idx in idx_list:
        x = torch.tensor(frames[idx], dtype=torch.float64) / 255.0
        w1, b1, w2, b2, f1, fb1, f2, fb2 = params
        h = torch.relu(torch.nn.functional.conv2d(x, w1, b1, stride=2))
        h = torch.relu(torch.nn.functional.conv2d(h, w2, b2, stride=1))
        h = h.permute(0, 2, 3, 1).reshape(len(idx), -1)
        h = torch.relu(h @ f1 + fb1)
        out = h @ f2 + fb2
        A = out.shape[1] - 1
        logits, value = out[:, :A], out[:, A]
        logp_all = torch.log_softmax(logits, dim=-1)
        a = torch.tensor(actions[idx], dtype=torch.long)
        new_logp = logp_all.gather(1, a[:, None])[:, 0]
        ent = -(logp_all.exp() * logp_all).sum(dim=1)
        ratio = torch.exp(new_logp - torch.tensor(old_logp[idx]))
        adv = torch.tensor(adv_n[idx])
        surr = torch.minimum(ratio * adv, torch.clamp(ratio, 1 - cfg["clip_eps"], 1 + cfg["clip_eps"]) * adv)
        policy_loss = -surr.mean()
        ov, R = torch.tensor(old_v[idx]), torch.tensor(ret[idx])
        clipped = ov + torch.clamp(value - ov, -cfg["value_clip_eps"], cfg["value_clip_eps"])
        value_loss = 0.5 * torch.maximum((value - R) ** 2, (clipped - R) ** 2).mean()
        entropy = ent.mean()
        loss = policy_loss + cfg["value_coef"] * value_loss - cfg["entropy_coef"] * entropy
        opt.zero_grad()
        loss.backward()
        norm = float(torch.sqrt(sum((p.grad ** 2).sum() for p in params)))
        if norm > cfg["max_grad_norm"]:
            for p in params:
                p.grad *= cfg["max_grad_norm"] / (norm + 1e-6)
        opt.step()
        lr_ = (new_logp.detach().numpy() - old_logp[idx])
        steps.append(dict(loss=loss.item(), policy_loss=policy_loss.item(), value_loss=value_loss.item(),
                          entropy=entropy.item(), grad_norm=norm, approx_kl=float(np.mean(np.expm1(lr_) - lr_))))
    return [p.detach().numpy() for p in params], steps


@pytest.mark.parametrize("max_grad_norm", [0.05, 1e6])
def test_ppo_update_oracle_matches_torch(max_grad_norm):
    from oracle.ppo import gae, minibatch_indices, normalize_advantages, ppo_update

    rng = np.random.default_rng(11)
    A, T, N = 4, 4, 4
    net = _small_net(rng, A)
    rollout = {
        "obs": rng.integers(0, 256, (T, N, 4, 12, 12), dtype=np.uint8),
        "actions": rng.integers(0, A, (T, N)),
        "rewards": rng.choice([-1.0, 0.0, 1.0], (T, N)).astype(np.float32),
        "dones": (rng.random((T, N)) < 0.2).astype(np.float32),
        "values": rng.standard_normal((T, N)).astype(np.float32),
        "logp": (np.log(rng.uniform(0.1, 0.5, (T, N)))).astype(np.float32),
        "last_values": rng.standard_normal(N).astype(np.float32),
        "valid": np.ones((T, N), np.float32),
    }
    rollout["valid"][2, 1] = 0.0
    cfg = dict(lr=1e-3, adam_eps=1e-8, clip_eps=0.1, value_clip_eps=0.1, value_coef=0.5, entropy_coef=0.01,
               max_grad_norm=max_grad_norm)
    res = ppo_update(net, rollout, rng=np.random.default_rng(5), minibatch_size=4, epochs=2, **cfg)
    adv, ret = gae(rollout["rewards"], rollout["values"], rollout["dones"], rollout["last_values"], 0.99, 0.95,
                   rollout["valid"])
    adv_n, _, _ = normalize_advantages(adv, rollout["valid"])
    idx_list = minibatch_indices(rollout["valid"], 4, 2, np.random.default_rng(5))
    want_params, want_steps = _torch_update(net, rollout, idx_list, adv_n.reshape(-1),
                                            np.asarray(ret, np.float64).reshape(-1), cfg)
    assert len(res["steps"]) == len(want_steps) == 6
    for got, want in zip(res["steps"], want_steps):
        for k in want:
            assert got[k] == pytest.approx(want[k], rel=1e-9, abs=1e-12), k
    clipped = [s["grad_norm"] > max_grad_norm for s in res["steps"]]
    assert all(clipped) if max_grad_norm < 1 else not any(clipped)
    for got, want in zip(res["net"].flat(), want_params):
        assert np.allclose(got, want, rtol=1e-9, atol=1e-12)
