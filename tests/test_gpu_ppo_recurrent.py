"""The recurrent PPO update (ttrl/algos/ppo/recurrent.py:190-225,
ttrl/nets/recurrent.py, ttrl/buffers/seqbatch.py) on the GPU against the
float64 oracle (oracle/ppo.py: recurrent_ppo_update / recurrent_ppo_step,
pinned to torch): Nature-CNN trunk, GRU memory, 18- or 6-action policy head
and value head, sequence minibatches with episode-start resets inside
sequences, autoreset padding excluded from the loss.

Tolerances as the feedforward update's (tests/test_gpu_ppo_update.py): per
step loss terms, approx KL and gradient norm rel 1e-4; gradients and Adam
moments rel 1e-4 per tensor; parameters along a short trajectory rel 1e-4
except where Adam's direction is undecidable in fp32, and at the
recurrent-PPO shape step by step from the device's own state, with the
device's ReLU gates adopted inside the kink band."""

from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _rel(got, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


def _params(state: dict):
    from oracle.nets import QNet

    arrs = [np.asarray(v, np.float64) for v in state.values()]
    convs = [(arrs[2 * i], arrs[2 * i + 1].reshape(-1), s, 0) for i, s in enumerate((4, 2, 1))]
    trunk = QNet(convs, [(arrs[6], arrs[7].reshape(-1))], 1.0 / 255.0)
    gru = (arrs[8], arrs[9], arrs[10].reshape(-1), arrs[11].reshape(-1))
    head = (np.concatenate([arrs[12], arrs[14]], axis=1), np.concatenate([arrs[13].reshape(-1),
                                                                         arrs[15].reshape(-1)]))
    return dict(trunk=trunk, gru=gru, head=head)


def _flat(p: dict):
    return p["trunk"].flat() + list(p["gru"]) + list(p["head"])


def _per_param(learner, source):
    """Per-parameter device arrays (moments or grads) as a state-like dict in
    parameter order, conv weights OIHW."""
    from ttrl_amd.engine.conv import Conv2d, master_to_oihw
    from ttrl_amd.nets.acting import _walk_modules

    convs = {id(m.weight): m for _, m in _walk_modules(learner.net) if isinstance(m, Conv2d)}
    out = {}
    for i, (name, p) in enumerate(learner.net.named_parameters()):
        a = source(i, p).numpy().astype(np.float64).reshape(p.shape)
        m = convs.get(id(p))
        if m is not None:
            a = master_to_oihw(a, m._oihw_shape, m.input_layout)
        out[name] = a
    return out


def _learner(device, *, T, N, L, Hd, mb, epochs, mode, A, seed):
    from ttrl_amd.algos.ppo import PPOConfig, RecurrentConfig, RecurrentPPOLearner
    from ttrl_amd.spaces import ActionSpec, ObsSpec
    from ttrl_amd.workloads import he_uniform_qnet_state, recurrent_ppo_rollout

    cfg = PPOConfig(minibatch_size=mb, epochs=epochs, n_steps=T, step_mode=mode,
                    recurrent=RecurrentConfig(hidden_size=Hd, seq_len=L))
    learner = RecurrentPPOLearner(ObsSpec.image((4, 84, 84)), ActionSpec.discrete(A), device, cfg=cfg, seed=seed)
    state = he_uniform_qnet_state(learner.net, seed + 1)
    learner.net.load_state_dict(state)
    rollout = recurrent_ppo_rollout(seed + 2, T, N, A, L, Hd)
    rollout["dones"][T // 2] = 1.0  # resets inside sequences
    rollout["starts"][1:] = rollout["dones"][:-1]
    valid = np.ones((T, N), np.float32)
    valid[-2:, 0] = 0.0  # autoreset padding at the end of lane 0
    rollout["valid"] = valid
    return learner, cfg, learner.net.state_dict(), rollout


@pytest.mark.parametrize("mode", ["graph", "eager"])
def test_recurrent_update_matches_oracle_small(device, mode):
    from oracle.ppo import recurrent_ppo_update
    from ttrl_amd.algos.ppo import PPOLearner

    T, N, L, Hd, mb, A, seed = 16, 4, 8, 32, 16, 6, 41
    learner, cfg, state, rollout = _learner(device, T=T, N=N, L=L, Hd=Hd, mb=mb, epochs=2, mode=mode, A=A,
                                           seed=seed)
    try:
        m = learner.update(rollout)
        steps = int(m["minibatches"])
        ring = learner._res.ring.numpy()[:steps]
        got = _params(learner.net.state_dict())
    finally:
        learner.close()
    ref = recurrent_ppo_update(_params(state), rollout, rng=np.random.default_rng(seed), minibatch_size=mb,
                               epochs=2, seq_len=L, lr=cfg.lr, adam_eps=cfg.adam_eps,
                               max_grad_norm=cfg.max_grad_norm)
    assert steps == len(ref["steps"]) == 2 * ((T // L) * N // (mb // L))
    for k, key in enumerate(PPOLearner.METRICS):
        want = np.array([s[key] for s in ref["steps"]])
        assert np.all(np.abs(ring[:, k] - want) <= 1e-4 * np.maximum(np.abs(want), 1e-2)), (key, ring[:, k], want)
    for i, (g, w) in enumerate(zip(_flat(got), _flat(ref["params"]))):
        err = np.abs(g - w)
        big = err > 1e-4 * np.max(np.abs(w))
        # Adam (eps 1e-8) moves each entry by about lr * sign(S): an entry
        # whose float64 and fp32 S straddle 0 may differ by up to 2 lr per
        # step; such entries must stay rare.
        assert np.all(err[big] <= 2 * cfg.lr * steps), i
        assert big.mean() < 0.01, (i, float(big.mean()))


@pytest.mark.parametrize("mode,epochs", [("eager", 1), ("graph", 4)])
def test_recurrent_minibatch_steps_at_the_config_shape_step_by_step(device, mode, epochs):
    """16 envs x 128 steps, sequences of 32, hidden 512, minibatches of 512
    rows (16 sequences), 18 actions, each step from the device's own
    parameters and Adam moments.  Eager: one epoch of four steps, each
    recording its ReLU outputs as it runs.  Graph (the form the benchmark
    times): the whole update, 4 epochs x 4 minibatches, as 16 replays of the
    captured step, the ReLU outputs read after each replay from the buffers
    the capture recorded."""
    from oracle.adam import fused_step
    from oracle.ppo import recurrent_ppo_step, recurrent_ppo_update
    from ttrl_amd.algos.ppo import PPOLearner
    from ttrl_amd.engine import layers as layers_mod

    T, N, L, Hd, mb, A, seed = 128, 16, 32, 512, 512, 18, 51
    learner, cfg, state, rollout = _learner(device, T=T, N=N, L=L, Hd=Hd, mb=mb, epochs=epochs, mode=mode, A=A,
                                           seed=seed)
    try:
        steps = learner.load_rollout(rollout)
        assert steps == 4 * epochs
        ref = recurrent_ppo_update(_params(state), rollout, rng=np.random.default_rng(seed), minibatch_size=mb,
                                   epochs=epochs, seq_len=L, lr=cfg.lr, adam_eps=cfg.adam_eps,
                                   max_grad_norm=cfg.max_grad_norm, batches_only=True)
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
        opt = learner.optimizer
        for t in range(steps):
            p0 = _params(learner.net.state_dict())
            S0 = _flat(_params(_per_param(learner, lambda i, p: opt.m[i])))
            V0 = _flat(_params(_per_param(learner, lambda i, p: opt.v[i])))
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
            r = recurrent_ppo_step(p0, S0, V0, t + 1, ref["batches"][t], seq_len=L, lr=cfg.lr,
                                   adam_eps=cfg.adam_eps, max_grad_norm=cfg.max_grad_norm, gates=gates)
            ring = learner._res.ring.numpy()[t]
            for k, key in enumerate(PPOLearner.METRICS):
                want = r["metrics"][key]
                assert abs(ring[k] - want) <= 1e-4 * max(abs(want), 1e-2), (t, key, ring[k], want)
            g_dev = _flat(_params(_per_param(learner, lambda i, p: p.grad)))
            for i, (g, w) in enumerate(zip(g_dev, r["grads"])):
                assert _rel(g, w) < 1e-4, (t, i)
            got = _flat(_params(learner.net.state_dict()))
            for i, q0 in enumerate(_flat(p0)):
                want, _, _ = fused_step(q0, g_dev[i], S0[i], V0[i], t + 1, cfg.lr, eps=cfg.adam_eps)
                assert _rel(got[i], want) < 1e-5, (t, i)
    finally:
        learner.close()
