"""Output heads (ttrl/nets/heads.py:25-116).  GaussianHead clamps log_std to
[-20, 2]; `forward` composes Linear + clamp like the reference, and
`forward_packed` computes both heads in one launch with the clamp in the
epilogue, returning [mean | log_std] rows for the fused squashed sample."""

from __future__ import annotations

import ctypes as C

from ttrl_amd import _lib
from ttrl_amd.engine.autograd import Tensor, _detached, _needs, relu_mask
from ttrl_amd.engine.layers import Linear
from ttrl_amd.engine.nn import Module, ModuleDict
from ttrl_amd.engine.ops import clamp
from ttrl_amd.engine.ops.fused import grad_targets
from ttrl_amd.engine.tensor import DeviceArray

LOG_STD_MIN = -20.0
LOG_STD_MAX = 2.0


class QHead(Module):
    def __init__(self, in_features: int, n_actions: int, device):
        self.q = Linear(in_features, n_actions, device)
        self.n_actions = int(n_actions)

    def forward(self, x):
        return self.q(x)


class CategoricalHead(Module):
    def __init__(self, in_features: int, n_actions: int, device):
        self.logits = Linear(in_features, n_actions, device)
        self.n_actions = int(n_actions)

    def forward(self, x):
        return self.logits(x)


class ValueHead(Module):
    def __init__(self, in_features: int, device):
        self.value = Linear(in_features, 1, device)

    def forward(self, x):
        return self.value(x)


class GaussianHead(Module):
    def __init__(self, in_features: int, action_dim: int, device, *, log_std_min: float = LOG_STD_MIN,
                 log_std_max: float = LOG_STD_MAX):
        if log_std_min >= log_std_max:
            raise ValueError(
                f"GaussianHead: log_std_min must be < log_std_max, got {log_std_min} and {log_std_max}"
            )
        self.action_dim = int(action_dim)
        self.log_std_min = float(log_std_min)
        self.log_std_max = float(log_std_max)
        self.heads = ModuleDict({
            "mean": Linear(in_features, self.action_dim, device),
            "log_std": Linear(in_features, self.action_dim, device),
        })

    def forward(self, x):
        mean = self.heads["mean"](x)
        log_std = clamp(self.heads["log_std"](x), self.log_std_min, self.log_std_max)
        return mean, log_std

    def forward_packed(self, x: Tensor) -> Tensor:
        """(B, 2d) rows [mean | clamp(log_std)] from one launch.  Its backward
        expects the log_std columns' gradient already masked to the open clamp
        interval, which the fused squashed-sample backward provides."""
        return packed_linear_pair(self.heads["mean"], self.heads["log_std"], x,
                                  clamp=(self.log_std_min, self.log_std_max), op="gaussian_head")


def policy_value_packed(policy: CategoricalHead, value: ValueHead, x: Tensor) -> Tensor:
    """(B, A + 1) rows [logits | value] of a shared-trunk actor-critic's two
    heads (ttrl/nets/models.py:65-71) from one launch."""
    return packed_linear_pair(policy.logits, value.value, x, op="policy_value_head")


def _packed_launch(first: Linear, second: Linear, x: DeviceArray, clamp) -> DeviceArray:
    """(M, n1 + n2) rows [x W1 + b1 | x W2 + b2] over every row of x, one launch."""
    M, K = (int(d) for d in x.shape)
    n1 = first.out_features
    N = n1 + second.out_features
    y = DeviceArray(x.dev, (M, N))
    desc = _lib.LinearDesc()
    desc.M, desc.K, desc.N, desc.groups = M, K, N, 1
    desc.x, desc.ldx = x.ptr, K
    desc.W, desc.b = first.weight.data.ptr, None if first.bias is None else first.bias.data.ptr
    desc.W2, desc.b2, desc.n1 = second.weight.data.ptr, None if second.bias is None else second.bias.data.ptr, n1
    desc.y = y.ptr
    if clamp is not None:
        desc.clamp_col, desc.lo, desc.hi = n1, float(clamp[0]), float(clamp[1])
    x.dev.call("ttrl_linear_forward", C.byref(desc))
    return y


def packed_tape(first: Linear, second: Linear, x: Tensor, y: DeviceArray, op: str) -> Tensor:
    """The tape node of a packed pair's rows: y (x's rows) computed elsewhere."""
    M, K = (int(d) for d in x.shape)
    n1 = first.out_features
    N = n1 + second.out_features
    dev = x.device
    params = tuple(t for t in (first.weight, first.bias, second.weight, second.bias) if t is not None)
    if not _needs(x, *params):
        return _detached(y)
    if first.bias is None or second.bias is None:
        raise ValueError(f"{op}: the fused backward needs both layers to have a bias")
    out = Tensor(y, True, (x,) + params, op)
    x_data = x.data

    def _backward(grad):
        (dw1, db1, dw2, db2), beta_w = grad_targets(*params)
        (dx,), beta_x = grad_targets(x)
        # x a ReLU output: its gate applied as dx is written, so the layer
        # below takes the gradient without a masking pass of its own
        xmask = relu_mask(x) if dx is not None else None
        b = _lib.LinearDesc()
        b.M, b.K, b.N, b.groups = M, K, N, 1
        b.x, b.ldx = x_data.ptr, K
        b.W, b.W2, b.n1 = first.weight.data.ptr, second.weight.data.ptr, n1
        b.dy = grad.ptr
        if dw1 is not None:
            b.dW, b.db, b.dW2, b.db2 = dw1.ptr, db1.ptr, dw2.ptr, db2.ptr
        b.dx = None if dx is None else dx.ptr
        b.dxmask = None if xmask is None else xmask.ptr
        b.lddx = K
        b.beta_w, b.beta_x = beta_w, beta_x
        dev.call("ttrl_linear_backward", C.byref(b))
        if dx is not None:
            x._note_write(beta_x, xmask is not None)

    out._backward = _backward
    return out


def packed_linear_pair(first: Linear, second: Linear, x: Tensor, *, clamp=None, op: str) -> Tensor:
    """(B, n1 + n2) rows [x W1 + b1 | x W2 + b2] of two Linear layers over one
    input, from one launch; `clamp` = (lo, hi) clamps the second block in the
    epilogue.  Backward: both layers' dW and db and dx in one launch."""
    return packed_tape(first, second, x, _packed_launch(first, second, x.data, clamp), op)


def packed_linear_pair_rows(first: Linear, second: Linear, x: Tensor, x_all: DeviceArray, *, clamp=None,
                            op: str):
    """packed_linear_pair over every row of x_all in one launch, the tape over
    its leading rows (x, whose data views them).  -> (tape node, y_all)."""
    B = int(x.shape[0])
    if x.data.ptr != x_all.ptr or int(x_all.shape[0]) < B:
        raise ValueError(f"{op}: x must view the leading rows of x_all")
    y_all = _packed_launch(first, second, x_all, clamp)
    N = int(y_all.shape[1])
    return packed_tape(first, second, x, y_all.view(0, (B, N)), op), y_all
