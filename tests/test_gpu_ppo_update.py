"""The PPO update (ttrl/algos/ppo/learn.py:46-112) on the GPU against the
float64 oracle (oracle/ppo.py:ppo_update): shared Nature-CNN trunk with an
18- or 6-action policy head and a value head, GAE (gamma 0.99, lambda 0.95),
advantage normalisation, the reference's shuffles, clip 0.1, value clip 0.1,
value coef 0.5, entropy coef 0.01, global-norm clip 0.5, Adam lr 2.5e-4.

Tolerances: every minibatch step's loss, policy loss, value loss, entropy,
approx_kl and pre-clip gradient norm, and every parameter tensor after the
update, within rel 1e-4 of the oracle (max abs error over the tensor
relative to its max |value|; a scalar relative to max(|value|, 1e-2))."""

from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _rel(got, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


def _to_oracle(state: dict):
    from oracle.nets import QNet

    items = list(state.items())
    pairs = [(np.asarray(items[i][1], np.float64), np.asarray(items[i + 1][1], np.float64).reshape(-1))
             for i in range(0, len(items), 2)]
    convs = [(w, b, s, 0) for (w, b), s in zip(pairs[:3], (4, 2, 1))]
    (fw, fb), (pw, pb), (vw, vb) = pairs[3:]
    head = (np.concatenate([pw, vw], axis=1), np.concatenate([pb, vb]))
    return QNet(convs, [(fw, fb), head], 1.0 / 255.0)


def _grads_state(learner) -> dict:
    """The current gradients in state_dict layout (conv weights OIHW)."""
    from ttrl_amd.engine.conv import Conv2d
    from ttrl_amd.nets.acting import _walk_modules

    convs = {id(m.weight): m for _, m in _walk_modules(learner.net) if isinstance(m, Conv2d)}
    out = {}
    for name, p in learner.net.named_parameters():
        m = convs.get(id(p))
        out[name] = m.weight_grad_numpy() if m is not None else p.grad.numpy().reshape(p.shape)
    return out


def _run(device, *, T, N, mb, epochs, mode, A, seed, valid_holes=0):
    from oracle.ppo import ppo_update
    from ttrl_amd.algos.ppo import PPOConfig, PPOLearner
    from ttrl_amd.spaces import ActionSpec, ObsSpec
    from ttrl_amd.workloads import he_uniform_qnet_state, ppo_rollout

    cfg = PPOConfig(minibatch_size=mb, epochs=epochs, step_mode=mode, n_steps=T)
    learner = PPOLearner(ObsSpec.image((4, 84, 84)), ActionSpec.discrete(A), device, cfg=cfg, seed=seed)
    try:
        state = he_uniform_qnet_state(learner.net, seed + 1)
        learner.net.load_state_dict(state)
        rollout = ppo_rollout(seed + 2, T, N, A)
        if valid_holes:
            valid = np.ones((T, N), np.float32)
            holes = np.random.default_rng(seed + 3).choice(T * N, valid_holes, replace=False)
            valid.reshape(-1)[holes] = 0.0
            rollout["valid"] = valid
        metrics = learner.update(rollout)
        steps = int(metrics["minibatches"])
        ring = learner._res.ring.numpy()[:steps]
        got_state = learner.net.state_dict()
        last_grads = _grads_state(learner)
    finally:
        learner.close()
    ref = ppo_update(_to_oracle(state), rollout, rng=np.random.default_rng(seed), minibatch_size=mb,
                     epochs=epochs, lr=cfg.lr, adam_eps=cfg.adam_eps, max_grad_norm=cfg.max_grad_norm,
                     keep_grads=True)
    assert steps == len(ref["steps"])
    for k, key in enumerate(PPOLearner.METRICS):
        want = np.array([s[key] for s in ref["steps"]])
        err = np.abs(ring[:, k] - want) / np.maximum(np.abs(want), 1e-2)
        assert np.all(err < 1e-4), (key, ring[:, k], want)
        assert metrics[key] == pytest.approx(float(np.mean(ring[:, k])), rel=1e-6)
    got_oracle = _to_oracle(got_state)
    for g, w in zip(_to_oracle(last_grads).flat(), ref["grads"][-1]):
        assert _rel(g, w) < 1e-4
    undecided_total = 0
    for i, (g, w) in enumerate(zip(got_oracle.flat(), ref["net"].flat())):
        undecided = np.zeros(w.shape, bool)
        for step in ref["grads"]:
            gt = np.abs(step[i])
            undecided |= gt <= 1e-5 * gt.max()
        err = np.abs(np.asarray(g, np.float64) - w)
        scale = np.max(np.abs(w))
        assert np.all(err[~undecided] <= 1e-4 * scale), (i, float(err[~undecided].max() / scale))
        assert np.all(err[undecided] <= 3 * cfg.lr * steps)
        undecided_total += int(undecided.sum())
    return metrics, undecided_total


@pytest.mark.parametrize("mode", ["graph", "eager"])
def test_ppo_update_matches_oracle_small(device, mode):
    m, undecided = _run(device, T=8, N=4, mb=16, epochs=2, mode=mode, A=6, seed=21, valid_holes=3)
    assert m["minibatches"] == 2.0 * (29 // 16)
    print(f"undecided Adam directions adopted: {undecided}")


def _adam_state(learner):
    """Device Adam moments (stored form) per parameter, in the oracle's
    layouts (conv weights OIHW)."""
    from ttrl_amd.engine.conv import Conv2d, master_to_oihw
    from ttrl_amd.nets.acting import _walk_modules

    convs = {id(m.weight): m for _, m in _walk_modules(learner.net) if isinstance(m, Conv2d)}
    opt = learner.optimizer
    S, V = [], []
    for i, p in enumerate(opt.params):
        m = convs.get(id(p))
        for store, out in ((opt.m[i], S), (opt.v[i], V)):
            a = store.numpy().astype(np.float64).reshape(p.shape)
            if m is not None:
                a = master_to_oihw(a, m._oihw_shape, m.input_layout)
            out.append(a.reshape(np.shape(a)))
    return S, V


def _flat_like_oracle(state_or_list):
    """Parameters (or per-parameter arrays) in the oracle's flat order: the
    two heads' blocks merged into one [logits | value] layer."""
    arrs = list(state_or_list.values()) if isinstance(state_or_list, dict) else list(state_or_list)
    arrs = [np.asarray(a, np.float64) for a in arrs]
    body, (pw, pb, vw, vb) = arrs[:-4], arrs[-4:]
    return body + [np.concatenate([pw, vw], axis=1), np.concatenate([pb.reshape(-1), vb.reshape(-1)])]


@pytest.mark.parametrize("mode,epochs", [("eager", 1), ("graph", 4)])
def test_ppo_minibatch_steps_at_256_match_oracle_step_by_step(device, mode, epochs):
    """The Atari PPO shape (8 envs x 128 steps, minibatches of 256, 18
    actions), compared step by step: before every step the oracle takes the
    device's parameters and Adam moments, so each step's arithmetic is
    checked from an identical state.  Eager: one epoch of four steps, each
    recording its ReLU outputs as it runs.  Graph: the whole update, 4 epochs
    x 4 minibatches, as 16 replays of the captured step; the ReLU outputs are
    read after each replay from the buffers the capture recorded.  The oracle
    adopts the device's gate only where its float64 pre-activation is within
    1e-4 of the tensor's RMS of zero (oracle.nets.gate)."""
    from ttrl_amd.engine import layers as layers_mod
    from oracle.ppo import ppo_minibatch_step, ppo_update
    from ttrl_amd.algos.ppo import PPOConfig, PPOLearner
    from ttrl_amd.spaces import ActionSpec, ObsSpec
    from ttrl_amd.workloads import he_uniform_qnet_state, ppo_rollout

    T, N, mb, A, seed = 128, 8, 256, 18, 31
    cfg = PPOConfig(minibatch_size=mb, epochs=epochs, n_steps=T, step_mode=mode)
    learner = PPOLearner(ObsSpec.image((4, 84, 84)), ActionSpec.discrete(A), device, cfg=cfg, seed=seed)
    try:
        state = he_uniform_qnet_state(learner.net, seed + 1)
        learner.net.load_state_dict(state)
        rollout = ppo_rollout(seed + 2, T, N, A)
        steps = learner.load_rollout(rollout)
        assert steps == 4 * epochs
        # The oracle's own pass, only for its minibatch rows and advantages.
        ref = ppo_update(_to_oracle(state), rollout, rng=np.random.default_rng(seed), minibatch_size=mb,
                         epochs=epochs, lr=cfg.lr, adam_eps=cfg.adam_eps, max_grad_norm=cfg.max_grad_norm)
        captured = None
        if mode == "graph":
            layers_mod.RECORD = []
            try:
                learner.begin_update()  # warm-up pass, then the capture: the last four records are the graph's
                captured = list(layers_mod.RECORD[-4:])
            finally:
                layers_mod.RECORD = None
            assert learner._graph is not None
        else:
            learner.begin_update()
        for t in range(steps):
            params0 = _to_oracle(learner.net.state_dict())
            S0, V0 = _adam_state(learner)
            if captured is not None:
                learner.run_steps(1)
                recs = [y.numpy() for y in captured]
            else:
                layers_mod.RECORD = []
                try:
                    learner.run_steps(1)
                    recs = [y.numpy() for y in layers_mod.RECORD[-4:]]
                finally:
                    layers_mod.RECORD = None
            shapes = [(mb, 20, 20, 32), (mb, 9, 9, 64), (mb, 7, 7, 64), (mb, 512)]
            gates = {n: y.reshape(sh) > 0 for n, y, sh in zip(("conv0", "conv1", "conv2", "fc0"), recs, shapes)}
            got_metrics = learner._res.ring.numpy()[t]
            r = ppo_minibatch_step(params0, _flat_like_oracle(S0), _flat_like_oracle(V0), t + 1, ref["batches"][t],
                                   lr=cfg.lr, adam_eps=cfg.adam_eps, max_grad_norm=cfg.max_grad_norm, gates=gates)
            for k, key in enumerate(PPOLearner.METRICS):
                want = r["metrics"][key]
                assert abs(got_metrics[k] - want) <= 1e-4 * max(abs(want), 1e-2), (t, key, got_metrics[k], want)
            for g, w in zip(_flat_like_oracle(_grads_state(learner)), r["grads"]):
                assert _rel(g, w) < 1e-4, t
            S1, V1 = _adam_state(learner)
            for g, w in zip(_flat_like_oracle(S1), r["S"]):
                assert _rel(g, w) < 1e-4, t
            for g, w in zip(_flat_like_oracle(V1), r["V"]):
                assert _rel(g, w) < 1e-4, t
            # Adam itself: the device's new parameters against the fused step
            # applied in float64 to the device's own gradients and moments
            # (eps 1e-8 makes the step about lr * sign(S), so the oracle's
            # gradients, equal to rel 1e-4 tensor-wide, cannot fix the
            # direction of entries whose S is within fp32 noise of 0).
            from oracle.adam import fused_step
            got = _flat_like_oracle(learner.net.state_dict())
            g_dev = _flat_like_oracle(_grads_state(learner))
            for i, p0 in enumerate(params0.flat()):
                want, _, _ = fused_step(p0, g_dev[i], _flat_like_oracle(S0)[i], _flat_like_oracle(V0)[i], t + 1,
                                        cfg.lr, eps=cfg.adam_eps)
                assert _rel(got[i], want) < 1e-5, (t, i)
    finally:
        learner.close()


def test_ppo_update_replays_across_updates(device):
    """A second update reuses the captured step (same rollout shape) and the
    step counters restart; a new shape recaptures."""
    from ttrl_amd.algos.ppo import PPOConfig, PPOLearner
    from ttrl_amd.spaces import ActionSpec, ObsSpec
    from ttrl_amd.workloads import ppo_rollout

    cfg = PPOConfig(minibatch_size=16, epochs=1, n_steps=8)
    learner = PPOLearner(ObsSpec.image((4, 84, 84)), ActionSpec.discrete(6), device, cfg=cfg, seed=3)
    try:
        m1 = learner.update(ppo_rollout(1, 8, 4, 6))
        g = learner._graph
        m2 = learner.update(ppo_rollout(2, 8, 4, 6))
        assert learner._graph is g and m1["minibatches"] == m2["minibatches"] == 2.0
        assert learner.optimizer.t == 4
        m3 = learner.update(ppo_rollout(3, 4, 8, 6))
        assert learner._graph is not g and m3["minibatches"] == 2.0
        assert all(np.isfinite(v) for v in m3.values())
        with pytest.raises(ValueError, match="zero minibatches"):
            learner.update(ppo_rollout(4, 2, 4, 6))
    finally:
        learner.close()
