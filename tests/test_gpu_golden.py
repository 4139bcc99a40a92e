"""The HIP path against the committed golden fixtures (tests/golden/),
independently of the live oracle: a padded strided convolution forward and
backward, the GAE scan (bit-exact), a PPO minibatch objective, and one DQN
learner update of the Nature CNN on 4x36x36 frames at batch 4.

Tolerances: conv rel 2e-5 of each tensor's scale; PPO and DQN rel 1e-4
(loss, mean_q, td_abs, grad norm; Adam deltas rel 1e-4 of the largest
delta, whose scale is the learning rate)."""

from __future__ import annotations

import ctypes as C
import importlib.util
from pathlib import Path

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"


def _load(name):
    with np.load(GOLDEN / name, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def _rel(got, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


def test_conv_small(device):
    from ttrl_amd import _lib
    from ttrl_amd.engine.conv import master_to_oihw, oihw_to_master
    from ttrl_amd.engine.tensor import DeviceArray, to_device
    g = _load("conv_small.npz")
    B, Cc, H, W, O, k, s, p = (int(v) for v in g["geom"])
    geom = _lib.ConvGeom(B, Cc, H, W, O, k, s, p, _lib.LAYOUT_NHWC_F32)
    xd = to_device(g["x"], device)
    wd = to_device(oihw_to_master(g["w"], "nhwc"), device)
    bd = to_device(g["b"], device)
    y = DeviceArray(device, g["y"].shape)
    device.call("ttrl_conv2d_forward", C.byref(geom), xd.vp, wd.vp, bd.vp, y.vp, C.c_float(1.0), 0)
    assert _rel(y.numpy(), g["y"]) < 2e-5
    dyd = to_device(g["dy"], device)
    dw = DeviceArray(device, wd.shape)
    db = DeviceArray(device, (O,))
    device.call("ttrl_conv2d_backward_weight", C.byref(geom), xd.vp, C.c_float(1.0), dyd.vp, None, dw.vp, db.vp,
                C.c_float(0.0))
    assert _rel(master_to_oihw(dw.numpy(), g["w"].shape, "nhwc"), g["dw"]) < 2e-5
    assert _rel(db.numpy(), g["db"]) < 2e-5
    dx = DeviceArray(device, g["x"].shape)
    device.call("ttrl_conv2d_backward_input", C.byref(geom), dyd.vp, None, wd.vp, dx.vp, None, C.c_float(1.0),
                C.c_float(0.0))
    assert _rel(dx.numpy(), g["dx"]) < 2e-5


def test_gae_rollout(device):
    from ttrl_amd.algos.ppo import compute_gae
    g = _load("gae_128x8.npz")
    adv, ret = compute_gae(device, g["rewards"], g["values"], g["dones"], g["last_values"], float(g["gamma"]),
                           float(g["lam"]), g["valid"])
    assert np.array_equal(adv.numpy(), g["advantages"])
    assert np.array_equal(ret.numpy(), g["returns"])


def test_ppo_minibatch(device):
    from ttrl_amd.algos.ppo import PPOLossConfig, objective
    from ttrl_amd.engine.autograd import Tensor
    g = _load("ppo_b64.npz")
    B = g["logits"].shape[0]
    logits = Tensor.from_numpy(g["logits"], device, requires_grad=True)
    value = Tensor.from_numpy(g["values"].reshape(B, 1), device, requires_grad=True)
    clip, vclip, vcoef, ecoef = (float(v) for v in g["cfg"])
    batch = dict(actions=g["actions"], old_logp=g["old_logp"], advantages=g["advantages"], returns=g["returns"],
                 values=g["old_values"])
    loss, parts, new_logp = objective(logits, value, batch, PPOLossConfig(clip, vclip, vcoef, ecoef),
                                      valid=g["valid"])
    loss.backward()
    got = [float(loss.numpy().reshape(-1)[0])] + [float(parts[k].numpy().reshape(-1)[0])
                                                  for k in ("policy_loss", "value_loss", "entropy")]
    for a, b in zip(got, g["loss"]):
        assert abs(a - b) < 1e-4 * max(abs(b), 1e-3)
    assert _rel(new_logp.numpy().reshape(-1), g["new_logp"]) < 1e-5
    assert _rel(logits.grad.numpy(), g["dlogits"]) < 1e-4
    assert _rel(value.grad.numpy().reshape(-1), g["dvalues"]) < 1e-4


def test_dqn_update_small(device):
    from ttrl_amd.algos.dqn import DQNConfig, DQNLearner
    from ttrl_amd.spaces import ActionSpec, ObsSpec
    spec = importlib.util.spec_from_file_location("make_golden", GOLDEN / "make_golden.py")
    mg = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mg)
    g = _load("dqn_b4_36.npz")
    online = mg.dqn_params(int(g["seed"]))
    assert mg.params_digest(online) == str(g["online_digest"])
    rng = np.random.default_rng(int(g["seed"]) + 1)
    target = [(p + 0.05 * np.abs(p).max() * rng.standard_normal(p.shape)).astype(np.float32) for p in online]
    assert mg.params_digest(target) == str(g["target_digest"])

    cfg = DQNConfig(lr=6.25e-5, adam_eps=1.5e-4, batch_size=4, step_mode="graph", double=True, prioritized=True)
    learner = DQNLearner(ObsSpec.image((4, 36, 36)), ActionSpec.discrete(6), device, cfg=cfg, seed=0)
    keys = list(learner.online.state_dict())
    shapes = {k: np.shape(v) for k, v in learner.online.state_dict().items()}
    learner.online.load_state_dict({k: p.reshape(shapes[k]) for k, p in zip(keys, online)})
    learner.target.load_state_dict({k: p.reshape(shapes[k]) for k, p in zip(keys, target)})
    batch = {k: g[k] for k in ("obs", "next_obs", "actions", "rewards", "dones", "discounts", "is_weights")}
    m = learner.update(batch)
    assert abs(m["loss"] - float(g["loss"])) <= 1e-4 * abs(float(g["loss"]))
    assert abs(m["mean_q"] - float(g["mean_q"])) <= 1e-4 * abs(float(g["mean_q"]))
    assert _rel(m["td_abs"], g["td_abs"]) < 1e-4
    assert abs(m["grad_norm"] - np.sqrt(float(g["grad_sq"]))) <= 1e-4 * np.sqrt(float(g["grad_sq"]))
    new = list(learner.online.state_dict().values())
    for i, (p1, p0) in enumerate(zip(new, online)):
        d = np.asarray(p1, np.float64).reshape(-1) - p0.astype(np.float64).reshape(-1)
        head = g[f"delta{i}_head"]
        # the delta of a float32 parameter is resolved to its ulp: compare at
        # the float32 spacing of the parameter plus rel 1e-4 of the step
        tol = 1e-4 * np.abs(head).max() + np.spacing(np.abs(p0.reshape(-1)[:head.size]).astype(np.float32)).max()
        assert np.max(np.abs(d[:head.size] - head)) <= tol, i
    learner.close()
