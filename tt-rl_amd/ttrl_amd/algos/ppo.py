"""PPO's device-side arithmetic behind the reference's interfaces.

compute_gae            RolloutBuffer.compute_gae (ttrl/buffers/rollout.py:195-226):
                       one lane per env, reverse scan, on the device
normalize_advantages   the minibatch advantage normalisation
                       (ttrl/buffers/rollout.py:269-270)
objective              the clipped-ratio objective with the categorical head's
                       log-prob and entropy (ttrl/algos/ppo/loss.py:42-83,
                       ttrl/algos/ppo/policy.py:64-76) as one fused tape node
                       whose backward writes d loss / d logits and d loss /
                       d values
clip_grad_norm         the global-norm clip (ttrl/algos/grads.py:13-43) over a
                       flat gradient arena, with no host read, so it can sit
                       inside a captured update

All of it runs on libttrl_hip; there is no host fallback.
"""

from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from ttrl_amd.engine.autograd import Tensor, _detached, _needs
from ttrl_amd.engine.tensor import DeviceArray, arena_of, to_device

__all__ = ["PPOLossConfig", "compute_gae", "normalize_advantages", "objective", "clip_grad_norm",
           "clip_grad_norm_device"]


def _dev(x, device, dtype=np.float32) -> DeviceArray:
    if isinstance(x, Tensor):
        return x.data
    if isinstance(x, DeviceArray):
        return x
    return to_device(np.ascontiguousarray(np.asarray(x, dtype)), device, dtype)


def compute_gae(device, rewards, values, dones, last_values, gamma: float, lam: float, valid=None):
    """-> (advantages, returns) as [T, N] device arrays.

    rewards, values, dones (and valid) are time-major [T, N]; last_values is
    the critic's value after the last step, [N].  Host arrays are uploaded;
    device arrays are used in place.
    """
    r = _dev(rewards, device)
    if len(r.shape) != 2:
        raise ValueError(f"compute_gae: rewards must be [T, N], got shape {r.shape}")
    T, N = (int(d) for d in r.shape)
    arrays = {"values": _dev(values, device), "dones": _dev(dones, device)}
    if valid is not None:
        arrays["valid"] = _dev(valid, device)
    for name, a in arrays.items():
        if tuple(a.shape) != (T, N):
            raise ValueError(f"compute_gae: {name} has shape {a.shape}, expected {(T, N)}")
    lv = _dev(last_values, device)
    if lv.numel != N:
        raise ValueError(f"compute_gae: last_values must have {N} entries, got {lv.numel}")
    adv = DeviceArray(device, (T, N))
    ret = DeviceArray(device, (T, N))
    device.call("ttrl_gae", T, N, r.vp, arrays["values"].vp, arrays["dones"].vp,
                arrays["valid"].vp if "valid" in arrays else None, lv.vp, C.c_double(gamma), C.c_double(lam),
                adv.vp, ret.vp)
    return adv, ret


def normalize_advantages(device, advantages, valid=None, eps: float = 1e-8):
    """-> (normalised advantages, stats [mean, std]) as device arrays."""
    a = _dev(advantages, device)
    out = DeviceArray(device, a.shape)
    stats = DeviceArray(device, (2,))
    v = None if valid is None else _dev(valid, device)
    if v is not None and v.numel != a.numel:
        raise ValueError(f"normalize_advantages: valid has {v.numel} entries, advantages {a.numel}")
    device.call("ttrl_normalize_advantages", a.vp, None if v is None else v.vp, C.c_long(a.numel),
                C.c_float(eps), out.vp, stats.vp)
    return out, stats


@dataclass(frozen=True)
class PPOLossConfig:
    """The objective's coefficients (ttrl/algos/ppo/config.py:75-78)."""

    clip_eps: float = 0.1
    value_clip_eps: float = 0.1
    value_coef: float = 0.5
    entropy_coef: float = 0.01

    def __post_init__(self):
        if not self.clip_eps > 0.0:
            raise ValueError(f"PPOLossConfig: clip_eps must be > 0, got {self.clip_eps}")
        if not self.value_clip_eps > 0.0:
            raise ValueError(f"PPOLossConfig: value_clip_eps must be > 0, got {self.value_clip_eps}")


def objective(policy_out: Tensor, value: Tensor, batch, cfg: PPOLossConfig, valid=None):
    """`(loss, parts, new_logp)` for one minibatch, as ttrl/algos/ppo/loss.py:42-83.

    policy_out: logits [B, A]; value: [B, 1]; `batch` carries `actions`,
    `old_logp`, `advantages`, `returns` and `values` (host arrays or device
    arrays of B entries).  `valid` ([B], optional) gives the masked mean of
    the recurrent path (masked_mean, loss.py:27-39); without it every row
    counts.  `loss` is a (1, 1) tape node differentiable in policy_out and
    value; `parts` holds detached policy_loss, value_loss and entropy.
    """
    dev = policy_out.device
    if len(policy_out.shape) != 2:
        raise ValueError(f"objective: policy_out must be [B, A], got {policy_out.shape}")
    B, A = (int(d) for d in policy_out.shape)
    if value.data.numel != B:
        raise ValueError(f"objective: value has {value.data.numel} entries, expected {B}")

    def field(name, dtype=np.float32):
        x = batch[name] if isinstance(batch, dict) else getattr(batch, name)
        arr = _dev(np.asarray(x).reshape(-1) if not isinstance(x, (DeviceArray, Tensor)) else x, dev, dtype)
        if arr.numel != B:
            raise ValueError(f"objective: batch.{name} has {arr.numel} entries, expected {B}")
        return arr

    actions = field("actions", np.int32)
    old_logp, adv, ret, old_v = (field(n) for n in ("old_logp", "advantages", "returns", "values"))
    w = None if valid is None else _dev(valid, dev)
    out4 = DeviceArray(dev, (4,))
    new_logp = DeviceArray(dev, (B, 1))
    dlogits = DeviceArray(dev, (B, A))
    dvalue = DeviceArray(dev, tuple(int(d) for d in value.shape))
    dev.call("ttrl_ppo_loss", B, A, policy_out.data.vp, actions.vp, old_logp.vp, adv.vp, ret.vp, old_v.vp,
             value.data.vp, None if w is None else w.vp, C.c_float(cfg.clip_eps), C.c_float(cfg.value_clip_eps),
             C.c_float(cfg.value_coef), C.c_float(cfg.entropy_coef), out4.vp, new_logp.vp, dlogits.vp, dvalue.vp)
    loss_arr = out4.view(0, (1, 1))
    parts = {"policy_loss": Tensor(out4.view(1, (1, 1))), "value_loss": Tensor(out4.view(2, (1, 1))),
             "entropy": Tensor(out4.view(3, (1, 1)))}
    if not _needs(policy_out, value):
        return _detached(loss_arr), parts, Tensor(new_logp)
    loss = Tensor(loss_arr, True, (policy_out, value), "ppo_objective")

    def _backward(grad):
        from ttrl_amd.engine.ops import _kernels as K

        scale = None if grad.unit else grad.reshape((1, 1))
        for t, g in ((policy_out, dlogits), (value, dvalue)):
            if t.requires_grad:
                t._accumulate(g if scale is None else K.binary("mul", g, scale))

    loss._backward = _backward
    return loss, parts, Tensor(new_logp)


def clip_grad_norm_device(grad: DeviceArray, max_norm: float) -> DeviceArray:
    """Clip one flat gradient buffer in place; -> the norm before clipping,
    as a (1,) device array (readable after the update)."""
    if not max_norm > 0.0:
        raise ValueError(f"clip_grad_norm: max_norm must be > 0, got {max_norm}")
    dev = grad.dev
    sq = DeviceArray(dev, (1,))
    norm = DeviceArray(dev, (1,))
    dev.call("ttrl_clip_grad_norm", grad.vp, C.c_long(grad.numel), C.c_float(max_norm), sq.vp, norm.vp)
    return norm


def clip_grad_norm(params, max_norm: float) -> float:
    """Scale every gradient so their global L2 norm is at most `max_norm`;
    returns the norm before clipping (ttrl/algos/grads.py:26-43).  The
    parameters must be exactly one arena's, each holding this step's
    gradient in its slot."""
    params = list(params)
    arena = arena_of(params)
    if arena is None:
        raise ValueError("clip_grad_norm: the parameters must be exactly one ParamArena's tensors, in order")
    if any(p.grad is None for p in params):
        raise RuntimeError("clip_grad_norm: every parameter of the arena needs this step's gradient")
    norm = clip_grad_norm_device(arena.grad, max_norm)
    return float(norm.numpy()[0])
