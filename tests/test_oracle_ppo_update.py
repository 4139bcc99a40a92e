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


def test_sequence_minibatches_follow_the_reference_rule():
    """Whole sequences over (chunk, lane), one permutation per epoch, rows
    time-major (ttrl/buffers/seqbatch.py:52-76, ttrl/buffers/sequences.py:121-155)."""
    from oracle.ppo import sequence_minibatches

    T, N, L, mb = 8, 3, 4, 8
    got = sequence_minibatches(T, N, L, mb, 2, np.random.default_rng(1))
    rng = np.random.default_rng(1)
    total, S = (T // L) * N, mb // L
    k = 0
    for _ in range(2):
        perm = rng.permutation(total)
        for start in range(0, (total // S) * S, S):
            ids = perm[start:start + S]
            rows, h0 = got[k]
            k += 1
            for s, i in enumerate(ids):
                chunk, lane = divmod(int(i), N)
                assert h0[s] == chunk * N + lane
                for t in range(L):
                    assert rows[t * S + s] == (chunk * L + t) * N + lane  # one lane, consecutive steps
    assert k == len(got) == 2 * (total // S)


def test_recurrent_ppo_oracle_matches_torch():
    import torch

    from oracle.ppo import gae, normalize_advantages, recurrent_ppo_update, sequence_minibatches

    torch.set_default_dtype(torch.float64)
    rng = np.random.default_rng(21)
    A, T, N, L, Hd, mb = 4, 8, 2, 4, 6, 8
    base = _small_net(rng, 16 - 1)  # convs and fc1 (72 -> 16); the head below replaces its last layer
    from oracle.nets import QNet
    trunk = QNet(base.convs, [base.fcs[0]], base.scale)
    u = lambda *s: rng.uniform(-0.4, 0.4, s)
    gru = (u(16, 3 * Hd), u(Hd, 3 * Hd), u(3 * Hd), u(3 * Hd))
    head = (u(Hd, A + 1), u(A + 1))
    rollout = {
        "obs": rng.integers(0, 256, (T, N, 4, 12, 12), dtype=np.uint8),
        "actions": rng.integers(0, A, (T, N)),
        "rewards": rng.choice([-1.0, 0.0, 1.0], (T, N)).astype(np.float32),
        "dones": (rng.random((T, N)) < 0.2).astype(np.float32),
        "values": rng.standard_normal((T, N)).astype(np.float32),
        "logp": np.log(rng.uniform(0.1, 0.5, (T, N))).astype(np.float32),
        "last_values": rng.standard_normal(N).astype(np.float32),
        "valid": np.ones((T, N), np.float32),
        "starts": (rng.random((T, N)) < 0.25).astype(np.float32),
        "hidden": rng.standard_normal((T // L, N, Hd)).astype(np.float32),
    }
    rollout["valid"][3, 1] = 0.0
    cfg = dict(lr=1e-3, adam_eps=1e-8, clip_eps=0.1, value_clip_eps=0.1, value_coef=0.5, entropy_coef=0.01,
               max_grad_norm=0.05)
    res = recurrent_ppo_update(dict(trunk=trunk, gru=gru, head=head), rollout, rng=np.random.default_rng(5),
                               minibatch_size=mb, epochs=2, seq_len=L, **cfg)

    params = [torch.tensor(p, requires_grad=True) for p in trunk.flat() + list(gru) + list(head)]
    opt = torch.optim.Adam(params, lr=cfg["lr"], eps=cfg["adam_eps"])
    adv, ret = gae(rollout["rewards"], rollout["values"], rollout["dones"], rollout["last_values"], 0.99, 0.95,
                   rollout["valid"])
    adv_n, _, _ = normalize_advantages(adv, rollout["valid"])
    flat_obs = rollout["obs"].reshape(T * N, 4, 12, 12)
    hid = rollout["hidden"].reshape(-1, Hd)
    for step, (rows, h0_rows) in enumerate(sequence_minibatches(T, N, L, mb, 2, np.random.default_rng(5))):
        w1, b1, w2, b2, f1, fb1, Wi, Wr, bi, br, Wo, bo = params
        x = torch.tensor(flat_obs[rows], dtype=torch.float64) / 255.0
        h = torch.relu(torch.nn.functional.conv2d(x, w1, b1, stride=2))
        h = torch.relu(torch.nn.functional.conv2d(h, w2, b2, stride=1))
        feat = torch.relu(h.permute(0, 2, 3, 1).reshape(len(rows), -1) @ f1 + fb1)
        S = mb // L
        seq = feat.reshape(L, S, -1)
        starts = torch.tensor(rollout["starts"].reshape(-1)[rows], dtype=torch.float64).reshape(L, S, 1)
        st = torch.tensor(hid[h0_rows])
        outs = []
        for t in range(L):
            st = st * (1 - starts[t])
            gi, gh = seq[t] @ Wi + bi, st @ Wr + br
            r = torch.sigmoid(gi[:, :Hd] + gh[:, :Hd])
            z = torch.sigmoid(gi[:, Hd:2 * Hd] + gh[:, Hd:2 * Hd])
            n = torch.tanh(gi[:, 2 * Hd:] + r * gh[:, 2 * Hd:])
            st = (1 - z) * n + z * st
            outs.append(st)
        out = torch.stack(outs).reshape(L * S, Hd) @ Wo + bo
        logits, value = out[:, :A], out[:, A]
        valid = torch.tensor(rollout["valid"].reshape(-1)[rows], dtype=torch.float64)
        keep = valid > 0
        old = torch.where(keep, torch.tensor(rollout["logp"].reshape(-1)[rows], dtype=torch.float64), 0.0)
        a_ = torch.tensor(adv_n.reshape(-1)[rows])
        R = torch.tensor(np.asarray(ret, np.float64).reshape(-1)[rows])
        a_, R = torch.where(keep, a_, 0.0), torch.where(keep, R, 0.0)
        ov = torch.tensor(rollout["values"].reshape(-1)[rows], dtype=torch.float64)
        logp_all = torch.log_softmax(logits, dim=-1)
        new_logp = logp_all.gather(1, torch.tensor(rollout["actions"].reshape(-1)[rows])[:, None])[:, 0]
        ratio = torch.exp(new_logp - old)
        surr = torch.minimum(ratio * a_, torch.clamp(ratio, 0.9, 1.1) * a_)
        total = valid.sum()
        pol = -(surr * valid).sum() / total
        clipped = ov + torch.clamp(value - ov, -0.1, 0.1)
        vl = 0.5 * (torch.maximum((value - R) ** 2, (clipped - R) ** 2) * valid).sum() / total
        ent = ((-(logp_all.exp() * logp_all).sum(1)) * valid).sum() / total
        loss = pol + 0.5 * vl - 0.01 * ent
        opt.zero_grad()
        loss.backward()
        norm = float(torch.sqrt(sum((p.grad ** 2).sum() for p in params)))
        if norm > cfg["max_grad_norm"]:
            for p in params:
                p.grad *= cfg["max_grad_norm"] / (norm + 1e-6)
        opt.step()
        got = res["steps"][step]
        assert got["loss"] == pytest.approx(loss.item(), rel=1e-9, abs=1e-12)
        assert got["grad_norm"] == pytest.approx(norm, rel=1e-9)
        lr_ = new_logp.detach().numpy() - old.numpy()
        assert got["approx_kl"] == pytest.approx(float(np.mean(np.expm1(lr_) - lr_)), rel=1e-9, abs=1e-12)
    want = [p.detach().numpy() for p in params]
    flat = res["params"]["trunk"].flat() + list(res["params"]["gru"]) + list(res["params"]["head"])
    for g, w in zip(flat, want):
        assert np.allclose(g, w, rtol=1e-9, atol=1e-12)
