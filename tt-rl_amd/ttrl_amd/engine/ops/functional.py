"""Composed blocks: huber, log_softmax, entropy, one-hot gather, masks and
the non-finite guard (ttrl/engine/ops/functional.py:40-195).  Each is built
from the primitive ops, exactly as the reference composes them."""

from __future__ import annotations

import numpy as np

from ttrl_amd.engine.autograd import Tensor
from ttrl_amd.engine.ops import _kernels as K
from ttrl_amd.engine.ops.elementwise import add, mul, sub
from ttrl_amd.engine.ops.reduce import max_dim_detached, sum_dim
from ttrl_amd.engine.ops.select import minimum
from ttrl_amd.engine.ops.unary import abs_, exp, log
from ttrl_amd.engine.tensor import DeviceArray


def apply_done_mask(value: Tensor, done: Tensor) -> Tensor:
    """value * (1 - done)."""
    return mul(value, sub(1.0, done))


masks = apply_done_mask


def huber(pred: Tensor, target: Tensor, delta: float = 1.0) -> Tensor:
    """Elementwise Huber loss through the clipped-quadratic identity, unreduced."""
    absdiff = abs_(sub(pred, target))
    quad = minimum(absdiff, delta)
    lin = sub(absdiff, quad)
    return add(mul(mul(quad, quad), 0.5), mul(lin, delta))


def purge_lane_caches(device) -> None:
    """No lane constants are cached (the one-hot kernel indexes directly)."""


def one_hot_host(indices, num_classes: int, device, dtype=None) -> Tensor:
    """(B,) host integer ids -> (B, num_classes) one-hot Tensor (uploads)."""
    idx = np.asarray(indices).reshape(-1).astype(np.int64)
    onehot = np.zeros((idx.shape[0], num_classes), dtype=np.float32)
    onehot[np.arange(idx.shape[0]), idx] = 1.0
    return Tensor.from_numpy(onehot, device, requires_grad=False)


def one_hot_device(indices: Tensor, num_classes: int) -> Tensor:
    """(B, 1) device float ids -> (B, num_classes): onehot[b, c] = (c - idx[b] == 0)."""
    batch = int(indices.shape[0])
    y = DeviceArray(indices.device, (batch, int(num_classes)))
    indices.device.call("ttrl_one_hot", indices.data.vp, y.vp, batch, int(num_classes))
    return Tensor(y, requires_grad=False)


def gather_onehot(values: Tensor, onehot: Tensor) -> Tensor:
    """sum(values * onehot, dim=-1, keepdim=True), differentiable in `values`."""
    return sum_dim(mul(values, onehot), dim=-1, keepdim=True)


def one_hot_gather(values: Tensor, indices, num_classes: int) -> Tensor:
    """values[b, indices[b]] for each row b, (B, 1)."""
    if isinstance(indices, Tensor):
        batch = int(indices.shape[0])
        onehot = one_hot_device(indices, num_classes)
    else:
        idx = np.asarray(indices).reshape(-1)
        batch = int(idx.shape[0])
        onehot = one_hot_host(idx, num_classes, values.device)
    if int(values.shape[0]) != batch:
        raise ValueError(f"one_hot_gather: values has batch {values.shape[0]}, indices has {batch}")
    return gather_onehot(values, onehot)


def log_softmax(x: Tensor, dim: int = -1) -> Tensor:
    """(x - m) - log(sum(exp(x - m))), m = detached max."""
    shifted = sub(x, max_dim_detached(x, dim=dim, keepdim=True))
    sum_exp = sum_dim(exp(shifted), dim=dim, keepdim=True)
    return sub(shifted, log(sum_exp))


def entropy(logits: Tensor, dim: int = -1) -> Tensor:
    """Categorical entropy from logits, one value per row (keepdim)."""
    logp = log_softmax(logits, dim=dim)
    return mul(sum_dim(mul(exp(logp), logp), dim=dim, keepdim=True), -1.0)


def non_finite_check(tensor) -> bool:
    """True if `tensor` holds any NaN or Inf (one host read)."""
    raw = tensor.data if isinstance(tensor, Tensor) else tensor
    finite = K.unary("isfinite", raw)
    bad = K.sum_all(K.unary("rsub_s", finite, 1.0))
    return bool(bad.numpy().reshape(-1)[0] > 0.0)
