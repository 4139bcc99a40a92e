"""Shared set-up of DQN parity tests: seeded learner + oracle networks."""

from __future__ import annotations

import numpy as np


def qnet_to_oracle(state: dict, scale: float = 1.0 / 255.0):
    """Module state_dict (in parameter order) -> oracle QNet."""
    from oracle.nets import QNet

    items = list(state.items())
    convs, fcs = [], []
    strides = [4, 2, 1]
    i = 0
    while i < len(items):
        k, w = items[i]
        _, b = items[i + 1]
        w = np.asarray(w, np.float64)
        b = np.asarray(b, np.float64).reshape(-1)
        if w.ndim == 4:
            convs.append((w, b, strides[len(convs)], 0))
        else:
            fcs.append((w, b))
        i += 2
    return QNet(convs, fcs, scale)


def oracle_to_state(net, keys) -> dict:
    flat = net.flat()
    return {k: v for k, v in zip(keys, flat)}


def build_learner(device, *, seed=0, step_mode="graph", double=True, batch=32, defer_grads=True):
    from ttrl_amd.algos.dqn import DQNConfig, DQNLearner
    from ttrl_amd.spaces import ActionSpec, ObsSpec
    from ttrl_amd.workloads import he_uniform_qnet_state

    cfg = DQNConfig(lr=6.25e-5, adam_eps=1.5e-4, batch_size=batch, step_mode=step_mode, double=double,
                    prioritized=True)
    learner = DQNLearner(ObsSpec.image((4, 84, 84)), ActionSpec.discrete(6), device, cfg=cfg, seed=seed,
                         defer_grads=defer_grads)
    online = he_uniform_qnet_state(learner.online, seed + 100)
    learner.online.load_state_dict(online)
    rng = np.random.default_rng(seed + 200)
    # target = online + jitter, so double and vanilla DQN disagree
    target = {k: (v + 0.05 * np.abs(v).max() * rng.standard_normal(v.shape)).astype(np.float32)
              for k, v in online.items()}
    learner.target.load_state_dict(target)
    return learner, online, target


def adam_moments(opt, module):
    """Adam's stored S and V per parameter in state_dict layout (conv OIHW)."""
    from ttrl_amd.engine.conv import Conv2d, master_to_oihw
    from ttrl_amd.nets.acting import _walk_modules

    convs = {id(m.weight): m for _, m in _walk_modules(module) if isinstance(m, Conv2d)}
    S, V = [], []
    for i, p in enumerate(opt.params):
        m = convs.get(id(p))
        for store, out in ((opt.m[i], S), (opt.v[i], V)):
            a = store.numpy().astype(np.float64).reshape(p.shape)
            out.append(master_to_oihw(a, m._oihw_shape, m.input_layout) if m is not None else a)
    return S, V
