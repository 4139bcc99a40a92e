"""Tanh-squashed diagonal Gaussian (ttrl/algos/gaussian.py:55-167,
ttrl/algos/sac/policy.py:22-59).

The composed spellings (`softplus`, `normal_logp`, `log_one_minus_tanh_sq`,
`squashed_logp`, `SquashedGaussian.sample`) build the reference's op graph
from primitive ops.  `squashed_sample` is the fused one-kernel version used
by the SAC learner: it takes the packed [mean | log_std] head rows and
returns the environment action and its log-density as two tape outputs that
share one backward kernel.
"""

from __future__ import annotations

import ctypes as C
import math

import numpy as np

from ttrl_amd.engine.autograd import Tensor, _needs
from ttrl_amd.engine.ops import abs_, add, div, exp, log, mul, neg, relu, square, sub, sum_dim, tanh
from ttrl_amd.engine.tensor import DeviceArray
from ttrl_amd.engine.ops import _kernels as K

__all__ = ["ActionScale", "LOG_2PI", "SquashedGaussian", "log_one_minus_tanh_sq", "normal_logp", "softplus",
           "squashed_logp", "squashed_logp_numpy", "squashed_sample"]

LOG_2PI = math.log(2.0 * math.pi)
_LOG_2 = math.log(2.0)


def softplus(x: Tensor) -> Tensor:
    """relu(x) + log(1 + exp(-|x|))."""
    return add(relu(x), log(add(exp(neg(abs_(x))), 1.0)))


def normal_logp(x: Tensor, mean: Tensor, log_std: Tensor) -> Tensor:
    dim = int(x.shape[-1])
    z = div(sub(x, mean), exp(log_std))
    per_dim = sub(mul(square(z), -0.5), log_std)
    return sub(sum_dim(per_dim, dim=-1, keepdim=True), 0.5 * dim * LOG_2PI)


def log_one_minus_tanh_sq(u: Tensor) -> Tensor:
    """2 * (log 2 - u - softplus(-2u))."""
    return mul(sub(sub(_LOG_2, u), softplus(mul(u, -2.0))), 2.0)


def squashed_logp(u: Tensor, mean: Tensor, log_std: Tensor) -> Tensor:
    correction = sum_dim(log_one_minus_tanh_sq(u), dim=-1, keepdim=True)
    return sub(normal_logp(u, mean, log_std), correction)


def squashed_logp_numpy(u, mean, log_std):
    z = (u - mean) / np.exp(log_std)
    normal = (-0.5 * z * z - log_std).sum(-1) - 0.5 * u.shape[-1] * LOG_2PI
    sp = np.maximum(-2.0 * u, 0.0) + np.log1p(np.exp(-np.abs(2.0 * u)))
    return (normal - (2.0 * (_LOG_2 - u - sp)).sum(-1)).astype(np.float32)


class ActionScale:
    """Affine map from [-1, 1]^d onto the action bounds, with its log-det."""

    def __init__(self, action_spec, device=None):
        low = action_spec.low_array
        high = action_spec.high_array
        self.dim = int(action_spec.dim)
        self.centre = ((high + low) * 0.5).astype(np.float32)
        self.half_width = ((high - low) * 0.5).astype(np.float32)
        self.log_det = float(np.sum(np.log(self.half_width.astype(np.float64))))
        self._scale = self._centre = None
        if device is not None:
            self._scale = Tensor.from_numpy(self.half_width.reshape(1, self.dim), device)
            self._centre = Tensor.from_numpy(self.centre.reshape(1, self.dim), device)

    def to_env(self, squashed: Tensor) -> Tensor:
        if self._scale is None:
            raise ValueError("ActionScale.to_env needs the device-resident bounds; construct it with a device")
        return add(mul(squashed, self._scale), self._centre)

    def env_logp(self, value: Tensor) -> Tensor:
        return sub(value, self.log_det)

    def to_env_numpy(self, squashed):
        return (self.centre + self.half_width * squashed).astype(np.float32)


class SquashedGaussian:
    """The reference's composed sample (ttrl/algos/sac/policy.py:30-40)."""

    def __init__(self, action_spec, device):
        self.action_spec = action_spec
        self.dim = int(action_spec.dim)
        self.scale = ActionScale(action_spec, device)

    def sample(self, mean: Tensor, log_std: Tensor, noise: Tensor):
        pre_squash = add(mean, mul(exp(log_std), noise))
        logp = self.scale.env_logp(squashed_logp(pre_squash, mean, log_std))
        return self.scale.to_env(tanh(pre_squash)), logp


class _HubOutput(Tensor):
    """An output of a multi-output op: its gradient is handed to the hub
    instead of being accumulated, and the hub runs one backward for all."""

    __slots__ = ("_hub", "_key")

    def _accumulate(self, grad):
        self._hub.grad[self._key].append(grad)

    def _accept_pair(self, g0, g1):
        self._hub.grad[self._key].extend((g0, g1))


def _sample_launch(head: DeviceArray, noise: DeviceArray, scale: ActionScale, action: DeviceArray,
                   logp: DeviceArray) -> DeviceArray:
    """ttrl_sac_sample over every row of `head`; -> u, the pre-squash sample."""
    rows, two_d = (int(s) for s in head.shape)
    d = two_d // 2
    if two_d != 2 * d or tuple(noise.shape) != (rows, d):
        raise ValueError(f"squashed_sample: head {head.shape} and noise {noise.shape} disagree")
    if scale._centre is None:
        raise ValueError("squashed_sample needs the device-resident bounds; construct ActionScale with a device")
    if logp.numel != rows or logp.dtype != np.float32 or action.numel != rows * d:
        raise ValueError(f"squashed_sample: outputs must hold {rows} rows")
    dev = head.dev
    u = DeviceArray(dev, (rows, d))
    dev.call("ttrl_sac_sample", rows, d, head.vp, noise.vp, scale._centre.data.vp, scale._scale.data.vp,
             C.c_float(scale.log_det), action.vp, logp.vp, u.vp)
    return u


def _sample_tape(head: Tensor, noise: DeviceArray, u: DeviceArray, action: DeviceArray, logp: DeviceArray,
                 scale: ActionScale, log_std_min: float, log_std_max: float):
    """The tape of one sample launch's rows: (action, logp) tensors whose
    backward is one ttrl_sac_sample_backward into `head`."""
    B, two_d = (int(s) for s in head.shape)
    d = two_d // 2
    dev = head.device
    half = scale._scale.data
    hub = Tensor(None, True, (head,), "squashed_sample")
    hub.grad = None
    outs = []
    for key, data in (("action", action), ("logp", logp)):
        t = _HubOutput(data, True, (hub,), f"sample_{key}")
        t._hub = hub
        t._key = key
        outs.append(t)
    parts = {"action": [], "logp": []}
    head_data = head.data

    def _arm(grad_holder=parts):
        hub.grad = grad_holder

    _arm()

    def _backward(parts_):
        ga = list(parts_["action"])
        gl = list(parts_["logp"])
        if not ga and not gl:
            return
        while len(ga) > 2:
            ga = [K.binary("add", ga[0], ga[1])] + ga[2:]
        while len(gl) > 1:
            gl = [K.binary("add", gl[0], gl[1])] + gl[2:]
        dh = DeviceArray(dev, (B, 2 * d))
        dev.call("ttrl_sac_sample_backward", B, d, head_data.vp, noise.vp, u.vp, half.vp,
                 ga[0].vp if ga else None, ga[1].vp if len(ga) > 1 else None, gl[0].vp if gl else None,
                 C.c_float(log_std_min), C.c_float(log_std_max), dh.vp, C.c_float(0.0))
        head._accumulate(dh)

    hub._backward = _backward
    return outs[0], outs[1]


def squashed_sample(head: Tensor, noise: Tensor, scale: ActionScale, log_std_min: float = -20.0,
                    log_std_max: float = 2.0, logp_out: DeviceArray | None = None):
    """One-kernel reparameterised sample from packed [mean | log_std] rows
    (log_std already clamped).  -> (action (B, d), logp (B, 1)).  `logp_out`
    may give the (B, 1) array the log-probabilities are written to."""
    B, two_d = (int(s) for s in head.shape)
    dev = head.device
    action = DeviceArray(dev, (B, two_d // 2))
    if logp_out is not None and (logp_out.numel != B or logp_out.dtype != np.float32):
        raise ValueError(f"squashed_sample: logp_out must hold {B} float32 values")
    logp = DeviceArray(dev, (B, 1)) if logp_out is None else logp_out.reshape((B, 1))
    u = _sample_launch(head.data, noise.data, scale, action, logp)
    if not _needs(head):
        return Tensor(action), Tensor(logp)
    return _sample_tape(head, noise.data, u, action, logp, scale, log_std_min, log_std_max)


def squashed_sample_rows(head: Tensor, head_all: DeviceArray, noise_all: DeviceArray, scale: ActionScale,
                         logp_all: DeviceArray, log_std_min: float = -20.0, log_std_max: float = 2.0):
    """squashed_sample over every row of `head_all` in one launch, the tape
    over its first B rows (`head`, a tape node whose data views them).
    -> (action, logp) tensors of the first B rows and (action, logp) arrays
    of the rest; `logp_all` receives every row's log-probability."""
    B = int(head.shape[0])
    rows, two_d = (int(s) for s in head_all.shape)
    d = two_d // 2
    if head.data.ptr != head_all.ptr or rows <= B:
        raise ValueError("squashed_sample_rows: head must view the leading rows of head_all")
    dev = head_all.dev
    action_all = DeviceArray(dev, (rows, d))
    u = _sample_launch(head_all, noise_all, scale, action_all, logp_all.reshape((rows, 1)))
    return sampled_rows_tape(head, action_all, logp_all, noise_all, u, scale, log_std_min, log_std_max)


def sampled_rows_tape(head: Tensor, action_all: DeviceArray, logp_all: DeviceArray, noise_all: DeviceArray,
                      u: DeviceArray, scale: ActionScale, log_std_min: float, log_std_max: float):
    """The tape of a sample already taken over every row (action_all,
    logp_all, the pre-squash u), over its first B rows (`head`'s).
    -> as squashed_sample_rows."""
    B = int(head.shape[0])
    rows, d = (int(s) for s in action_all.shape)
    action = action_all.view(0, (B, d))
    logp = logp_all.view(0, (B, 1))
    rest = (action_all.view(B * d, (rows - B, d)), logp_all.view(B, (rows - B, 1)))
    if not _needs(head):
        return Tensor(action), Tensor(logp), rest
    a, lp = _sample_tape(head, noise_all.view(0, (B, d)), u.view(0, (B, d)), action, logp, scale, log_std_min,
                         log_std_max)
    return a, lp, rest
