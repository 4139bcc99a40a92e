"""Pins of the oracle's SAC update: a torch float64 autograd restatement of
the reference's regions (ttrl/algos/sac/losses.py:25-94, step.py:63-96,
agent.py:218-238) with torch.optim.Adam, the log-density against
torch.distributions (Normal + the tanh change of variables), and central
finite differences of the sample's log-density."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import gaussian
from oracle.sac import SacParams, sac_update


def _params(seed, obs=5, act=2, hid=16):
    rng = np.random.default_rng(seed)

    def lin(i, o):
        b = np.sqrt(6 / i)
        return (rng.uniform(-b, b, (i, o)), rng.uniform(-1 / np.sqrt(i), 1 / np.sqrt(i), o))

    trunk = [lin(obs, hid), lin(hid, hid)]
    mean, log_std = lin(hid, act), lin(hid, act)
    critics = [[lin(obs + act, hid), lin(hid, hid), lin(hid, 1)] for _ in range(2)]
    targets = [[(w + 0.01 * rng.standard_normal(w.shape), b.copy()) for w, b in c] for c in critics]
    return SacParams(trunk, mean, log_std, critics, targets, log_alpha=float(rng.uniform(-0.5, 0.5)))


def _batch(seed, B=7, obs=5, act=2):
    from ttrl_amd.workloads import sac_batch
    b = sac_batch(seed, batch=B, obs_dim=obs, act_dim=act)
    b["dones"][1] = 1.0
    return b


def _T(a, grad=False):
    return torch.tensor(np.asarray(a, np.float64), requires_grad=grad)


def _torch_sac(P: SacParams, batch, lr=3e-4, eps=1e-8, tau=0.005):
    pol = [_T(x, True) for x in P.policy_flat()]
    crit = [_T(x, True) for x in P.critics_flat()]
    targ = [_T(x) for c in P.targets for pair in c for x in pair]
    log_alpha = _T([[P.log_alpha]], True)
    d = P.mean[0].shape[1]
    H = -float(d)

    def relu_clamp(x, lo, hi):
        lifted = torch.relu(x - lo) + lo
        return hi - torch.relu(hi - lifted)

    def policy(obs):
        h = obs
        for j in range(len(P.trunk)):
            h = torch.relu(h @ pol[2 * j] + pol[2 * j + 1])
        n = 2 * len(P.trunk)
        return h @ pol[n] + pol[n + 1], relu_clamp(h @ pol[n + 2] + pol[n + 3], -20.0, 2.0)

    def critic(ps, obs, a):
        h = torch.cat([obs, a], 1)
        for j in range(3):
            h = h @ ps[2 * j] + ps[2 * j + 1]
            if j < 2:
                h = torch.relu(h)
        return h[:, 0]

    def sample(mean, ls, noise):
        sigma = torch.exp(ls)
        u = mean + sigma * noise
        z = (u - mean) / sigma
        normal = (-0.5 * z * z - ls).sum(1) - 0.5 * d * math.log(2 * math.pi)
        sp = torch.relu(-2 * u) + torch.log(torch.exp(-torch.abs(-2 * u)) + 1)
        corr = (2 * (math.log(2) - u - sp)).sum(1)
        return torch.tanh(u), normal - corr

    obs, nxt = _T(batch["obs"]), _T(batch["next_obs"])
    alpha = float(np.exp(P.log_alpha))
    opt_c = torch.optim.Adam(crit, lr=lr, eps=eps)
    opt_p = torch.optim.Adam(pol, lr=lr, eps=eps)
    opt_a = torch.optim.Adam([log_alpha], lr=lr, eps=eps)
    with torch.no_grad():
        mn, lsn = policy(nxt)
        an, lpn = sample(mn, lsn, _T(batch["next_noise"]))
        q1t, q2t = critic(targ[:6], nxt, an), critic(targ[6:], nxt, an)
        soft = (q1t - torch.relu(q1t - q2t)) - lpn * alpha
        y = _T(batch["rewards"]) + soft * (1 - _T(batch["dones"])) * _T(batch["discounts"])
    act = _T(batch["actions"])
    loss_c = 0.5 * (((critic(crit[:6], obs, act) - y) ** 2).mean() + ((critic(crit[6:], obs, act) - y) ** 2).mean())
    loss_c.backward()
    cgrads = [p.grad.numpy().copy() for p in crit]
    opt_c.step()
    for p in crit:
        p.grad = None
    m, ls = policy(obs)
    a, lp = sample(m, ls, _T(batch["noise"]))
    q1, q2 = critic(crit[:6], obs, a), critic(crit[6:], obs, a)
    loss_a = (lp * alpha - (q1 - torch.relu(q1 - q2))).mean()
    loss_a.backward()
    pgrads = [p.grad.numpy().copy() for p in pol]
    opt_p.step()
    loss_al = -(log_alpha * (lp.detach() + H)).mean()
    loss_al.backward()
    opt_a.step()
    with torch.no_grad():
        new_t = [(1 - tau) * t + tau * c for t, c in zip(targ, crit)]
    return {
        "critic_loss": float(loss_c), "q_target": y.numpy(), "critic_grads": cgrads,
        "new_critics": [p.detach().numpy() for p in crit], "actor_loss": float(loss_a), "logp": lp.detach().numpy(),
        "policy_grads": pgrads, "new_policy": [p.detach().numpy() for p in pol], "alpha_loss": float(loss_al),
        "new_log_alpha": float(log_alpha.detach().numpy().reshape(-1)[0]), "new_targets": [t.numpy() for t in new_t],
    }


def test_sac_oracle_matches_torch_autograd():
    P = _params(0)
    batch = _batch(1)
    ref = sac_update(P, batch)
    tt = _torch_sac(P, batch)
    for k in ("critic_loss", "actor_loss", "alpha_loss", "new_log_alpha"):
        assert ref[k] == pytest.approx(tt[k], rel=1e-10, abs=1e-13), k
    np.testing.assert_allclose(ref["q_target"], tt["q_target"], rtol=1e-11)
    np.testing.assert_allclose(ref["logp"], tt["logp"], rtol=1e-11)
    for got, want in zip(ref["critic_grads"], tt["critic_grads"]):
        np.testing.assert_allclose(got.reshape(want.shape), want, rtol=1e-9, atol=1e-13)
    for got, want in zip(ref["policy_grads"], tt["policy_grads"]):
        np.testing.assert_allclose(got.reshape(want.shape), want, rtol=1e-9, atol=1e-13)
    crit_flat = [x for c in ref["new_critics"] for pair in c for x in pair]
    for got, want in zip(crit_flat, tt["new_critics"]):
        np.testing.assert_allclose(got.reshape(want.shape), want, rtol=1e-11, atol=1e-13)
    for got, want in zip(ref["new_policy"], tt["new_policy"]):
        np.testing.assert_allclose(got.reshape(want.shape), want, rtol=1e-11, atol=1e-13)
    targ_flat = [x for c in ref["new_targets"] for pair in c for x in pair]
    for got, want in zip(targ_flat, tt["new_targets"]):
        np.testing.assert_allclose(got.reshape(want.shape), want, rtol=1e-12, atol=1e-14)


def test_squashed_logp_matches_change_of_variables():
    rng = np.random.default_rng(2)
    mean, ls, eps = rng.standard_normal((6, 3)), rng.uniform(-2, 1, (6, 3)), rng.standard_normal((6, 3))
    a, logp, u = gaussian.sample(mean, ls, eps)
    normal = torch.distributions.Normal(torch.tensor(mean), torch.tensor(np.exp(ls)))
    ref = (normal.log_prob(torch.tensor(u)) - torch.log(1 - torch.tanh(torch.tensor(u)) ** 2)).sum(1).numpy()
    np.testing.assert_allclose(logp, ref, rtol=1e-10)
    np.testing.assert_allclose(a, np.tanh(u))


def test_sample_backward_finite_differences():
    rng = np.random.default_rng(3)
    mean, ls, eps = rng.standard_normal((4, 2)), rng.uniform(-1, 0.5, (4, 2)), rng.standard_normal((4, 2))
    ga, gl = rng.standard_normal((4, 2)), rng.standard_normal(4)

    def f(mu, s):
        a, lp, _ = gaussian.sample(mu, s, eps)
        return float(np.sum(a * ga) + np.sum(lp * gl))

    gm, gs = gaussian.sample_backward(mean, ls, eps, ga, gl)
    h = 1e-6
    for i in range(4):
        for j in range(2):
            dm = np.zeros_like(mean)
            dm[i, j] = h
            assert (f(mean + dm, ls) - f(mean - dm, ls)) / (2 * h) == pytest.approx(gm[i, j], rel=1e-6, abs=1e-9)
            assert (f(mean, ls + dm) - f(mean, ls - dm)) / (2 * h) == pytest.approx(gs[i, j], rel=1e-6, abs=1e-9)
