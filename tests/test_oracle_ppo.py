"""Pins of the oracle's PPO arithmetic: GAE against the reference test's
closed form (tests/buffers/test_rollout.py:17-55 of the reference) and its
padding known answer, the objective against a torch float64 autograd
restatement composed the way the reference composes it (exp of a log-prob
difference, minimum / maximum / clamp as relu identities,
ttrl/engine/ops/select.py:39-63, masked mean), log-softmax and entropy
against closed forms, and the global-norm clip against its definition."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import ppo


def _closed_form_gae(rewards, values, dones, last_values, gamma, lam):
    """A_t = sum_l (gamma*lam)^l delta_{t+l}, chain cut at a done (float64)."""
    T, N = rewards.shape
    out = np.zeros((T, N))
    for n in range(N):
        for t in range(T):
            acc, coef = 0.0, 1.0
            for l in range(t, T):
                nv = last_values[n] if l == T - 1 else values[l + 1][n]
                nd = 1.0 - dones[l][n]
                acc += coef * (rewards[l][n] + gamma * nv * nd - values[l][n])
                coef *= gamma * lam * nd
                if nd == 0.0:
                    break
            out[t, n] = acc
    return out


@pytest.mark.parametrize("seed", range(3))
def test_gae_matches_closed_form(seed):
    T, N, gamma, lam = 7, 3, 0.95, 0.9
    rng = np.random.default_rng(seed)
    r = rng.normal(size=(T, N)).astype(np.float32)
    v = rng.normal(size=(T, N)).astype(np.float32)
    d = (rng.random((T, N)) < 0.2).astype(np.float32)
    last = rng.normal(size=N).astype(np.float32)
    adv, ret = ppo.gae(r, v, d, last, gamma, lam)
    assert np.abs(adv - _closed_form_gae(r, v, d, last, gamma, lam)).max() < 1e-5
    assert np.abs(ret - (adv + v)).max() == 0.0


def test_gae_padding_cuts_the_chain():
    # The reference's known answer: gamma = lam = 1, reward 1, slot 2 padding.
    z = np.zeros((4, 1), np.float32)
    valid = np.array([[1], [1], [0], [1]], np.float32)
    adv, _ = ppo.gae(np.ones((4, 1), np.float32), z, z, np.zeros(1, np.float32), 1.0, 1.0, valid)
    assert adv.reshape(-1).tolist() == [2.0, 1.0, 0.0, 1.0]


def test_gae_double_product_rounding():
    # The reference multiplies by gamma*lam formed from two Python floats
    # (double), then rounded to float32; for gamma = lam = 0.9 that differs
    # from the product of the float32-rounded factors, so a float32 product
    # fails here.  With reward 1 at t = 1 and zero values, A_0 = gamma*lam.
    g, l = 0.9, 0.9
    assert np.float32(g * l) != np.float32(np.float32(g) * np.float32(l))
    z = np.zeros((2, 1), np.float32)
    adv, _ = ppo.gae(np.array([[0.0], [1.0]], np.float32), z, z, np.zeros(1, np.float32), g, l)
    assert adv[1, 0] == 1.0 and adv[0, 0] == np.float32(g * l)


def test_normalize_advantages():
    rng = np.random.default_rng(4)
    a = rng.normal(3.0, 2.0, (16, 4))
    valid = (rng.random((16, 4)) > 0.2).astype(np.float32)
    out, mean, std = ppo.normalize_advantages(a, valid)
    keep = valid > 0
    assert abs(out[keep].mean()) < 1e-12 and abs(out[keep].std() - std / (std + 1e-8)) < 1e-12
    assert np.all(out[~keep] == 0.0)
    assert abs(mean - a[keep].mean()) < 1e-12


def test_log_softmax_entropy_closed_forms():
    from scipy.special import logsumexp
    rng = np.random.default_rng(5)
    z = rng.normal(size=(9, 18)) * 3
    lp = ppo.log_softmax(z)
    assert np.abs(lp - (z - logsumexp(z, axis=1, keepdims=True))).max() < 1e-12
    p = np.exp(lp)
    assert np.abs(ppo.entropy(z) + (p * np.log(p)).sum(1)).max() < 1e-12
    assert abs(ppo.entropy(np.zeros((1, 18)))[0] - np.log(18)) < 1e-12  # uniform


def _torch_objective(z, a, old_lp, adv, ret, old_v, v, w, cfg):
    relu = torch.relu

    def minimum(x, y):
        return x - relu(x - y)

    def maximum(x, y):
        return x + relu(y - x)

    def clamp(x, lo, hi):
        return hi - relu(hi - (relu(x - lo) + lo))

    shifted = z - z.max(dim=1, keepdim=True).values.detach()
    lp_all = shifted - torch.log(torch.exp(shifted).sum(1, keepdim=True))
    onehot = torch.nn.functional.one_hot(torch.as_tensor(a), z.shape[1]).double()
    lp = (lp_all * onehot).sum(1)
    H = -(torch.exp(lp_all) * lp_all).sum(1)
    total = w.sum()

    def red(x):
        return (x * w).sum() / total

    ratio = torch.exp(lp - old_lp)
    surr = minimum(ratio * adv, clamp(ratio, 1 - cfg["clip_eps"], 1 + cfg["clip_eps"]) * adv)
    pl = -red(surr)
    vc = old_v + clamp(v - old_v, -cfg["value_clip_eps"], cfg["value_clip_eps"])
    eu, ec = v - ret, vc - ret
    vl = 0.5 * red(maximum(eu * eu, ec * ec))
    ent = red(H)
    return pl + vl * cfg["value_coef"] - cfg["entropy_coef"] * ent, pl, vl, ent, lp


@pytest.mark.parametrize("masked", [False, True])
def test_objective_matches_torch_autograd(masked):
    rng = np.random.default_rng(6 + masked)
    B, A = 64, 18
    cfg = dict(clip_eps=0.1, value_clip_eps=0.1, value_coef=0.5, entropy_coef=0.01)
    z = rng.normal(size=(B, A))
    a = rng.integers(0, A, B)
    lp0 = ppo.log_softmax(z)[np.arange(B), a]
    old_lp = lp0 + rng.normal(0, 0.15, B)  # ratios on both sides of the clip range
    adv = rng.normal(size=B)
    ret = rng.normal(size=B)
    old_v = rng.normal(size=B)
    v = old_v + rng.normal(0, 0.2, B)  # value deltas on both sides of the clip
    w = (rng.random(B) > 0.25).astype(np.float64) if masked else np.ones(B)
    got = ppo.ppo_objective(z, a, old_lp, adv, ret, old_v, v, w if masked else None, **cfg)
    zt = torch.tensor(z, requires_grad=True)
    vt = torch.tensor(v, requires_grad=True)
    loss, pl, vl, ent, lp = _torch_objective(zt, a, torch.tensor(old_lp), torch.tensor(adv), torch.tensor(ret),
                                             torch.tensor(old_v), vt, torch.tensor(w), cfg)
    loss.backward()
    for key, ref in (("loss", loss), ("policy_loss", pl), ("value_loss", vl), ("entropy", ent)):
        assert abs(got[key] - float(ref)) < 1e-12, key
    assert np.abs(got["new_logp"] - lp.detach().numpy()).max() < 1e-12
    assert np.abs(got["dlogits"] - zt.grad.numpy()).max() < 1e-12
    assert np.abs(got["dvalues"] - vt.grad.numpy()).max() < 1e-12


def test_objective_finite_differences():
    rng = np.random.default_rng(8)
    B, A = 6, 5
    cfg = dict(clip_eps=0.2, value_clip_eps=0.3, value_coef=0.5, entropy_coef=0.05)
    z = rng.normal(size=(B, A))
    a = rng.integers(0, A, B)
    old_lp = ppo.log_softmax(z)[np.arange(B), a] + rng.normal(0, 0.1, B)
    adv, ret, old_v = rng.normal(size=B), rng.normal(size=B), rng.normal(size=B)
    v = old_v + rng.normal(0, 0.1, B)

    def f(zz, vv):
        return ppo.ppo_objective(zz, a, old_lp, adv, ret, old_v, vv, **cfg)["loss"]

    g = ppo.ppo_objective(z, a, old_lp, adv, ret, old_v, v, **cfg)
    h = 1e-6
    for i, j in [(0, 0), (2, 3), (5, 4)]:
        dz = np.zeros_like(z)
        dz[i, j] = h
        fd = (f(z + dz, v) - f(z - dz, v)) / (2 * h)
        assert abs(fd - g["dlogits"][i, j]) < 1e-7
    for i in range(B):
        dv = np.zeros(B)
        dv[i] = h
        fd = (f(z, v + dv) - f(z, v - dv)) / (2 * h)
        assert abs(fd - g["dvalues"][i]) < 1e-7


def test_clip_grad_norm_definition():
    g = np.array([3.0, 4.0], np.float32)
    out, norm = ppo.clip_grad_norm(g, 1.0)
    assert norm == 5.0
    assert np.allclose(out, g * np.float32(1.0 / (5.0 + 1e-6)))
    out2, norm2 = ppo.clip_grad_norm(g, 10.0)
    assert norm2 == 5.0 and np.array_equal(out2, g)
