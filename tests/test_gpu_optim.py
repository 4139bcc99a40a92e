"""Adam on the GPU: the arena step against textbook Adam over several steps,
the checkpoint's canonical m and v (ttrl/engine/optim/checkpoint.py:15-104:
m = S(1-b1), v = V(1-b2)), and a resume from a state_dict continuing exactly
as the uninterrupted optimizer does.  Tolerance: rel 1e-6 (fp32 state vs
float64 textbook), exact equality for the resume."""

from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _net(device, seed):
    from ttrl_amd.engine.layers import Linear
    from ttrl_amd.engine.tensor import ParamArena
    rng = np.random.default_rng(seed)
    with ParamArena(device):
        l1 = Linear(37, 5, device)
        l2 = Linear(5, 3, device)
    params = list(l1.parameters()) + list(l2.parameters())
    init = [rng.uniform(-1, 1, p.shape).astype(np.float32) for p in params]
    for p, a in zip(params, init):
        p.data.upload(a.reshape(p.shape))
    return params, init


def _step(opt, params, grads, device):
    from ttrl_amd.engine.tensor import to_device
    opt.zero_grad()
    for p, g in zip(params, grads):
        p._accumulate(to_device(g.reshape(p.shape), device))
    opt.step()


def test_adam_state_dict_canonical_and_resume(device):
    from oracle import adam as oadam
    from ttrl_amd.engine.optim import Adam
    lr, b1, b2, eps = 1e-3, 0.9, 0.999, 1e-8
    params, init = _net(device, 0)
    opt = Adam(params, lr=lr, betas=(b1, b2), eps=eps)
    rng = np.random.default_rng(1)
    grads = [[rng.normal(0, 0.1, p.shape).astype(np.float32) for p in params] for _ in range(4)]
    ref = [(a.astype(np.float64), np.zeros(a.shape), np.zeros(a.shape)) for a in init]
    for t in range(1, 4):
        _step(opt, params, grads[t - 1], device)
        ref = [oadam.textbook_step(p, g, m, v, t, lr, b1, b2, eps) for (p, m, v), g in zip(ref, grads[t - 1])]
    sd = opt.state_dict()
    assert sd["t"] == 3
    for i, (p, m, v) in enumerate(ref):
        assert np.max(np.abs(params[i].numpy().reshape(p.shape) - p)) < 1e-6 * max(1.0, np.abs(p).max())
        assert np.max(np.abs(np.asarray(sd["m"][i]).reshape(m.shape) - m)) < 1e-6 * np.abs(m).max()
        assert np.max(np.abs(np.asarray(sd["v"][i]).reshape(v.shape) - v)) < 1e-6 * np.abs(v).max()

    # resume: a fresh optimizer over a copy of the parameters, loaded from the checkpoint
    params2, _ = _net(device, 0)
    for p2, p in zip(params2, params):
        p2.data.copy_from(p.data)
    opt2 = Adam(params2, lr=lr, betas=(b1, b2), eps=eps)
    opt2.load_state_dict(sd)
    _step(opt, params, grads[3], device)
    _step(opt2, params2, grads[3], device)
    for p, p2 in zip(params, params2):
        assert np.array_equal(p.numpy(), p2.numpy())
