"""`Linear`, `LayerNorm`, `ReLU`, `Tanh`, `Sequential`, `Flatten`
(ttrl/engine/layers.py:19-200).

Same constructors, parameter names, storage ((in, out) weights, (1, out)
biases) and init draws as the reference.  `Sequential` runs a layer that is
followed by a `ReLU` as one fused kernel (GEMM or convolution with a
bias+ReLU epilogue); the result equals running the two layers in turn.
"""

from __future__ import annotations

import math

import numpy as np

from ttrl_amd.engine.autograd import Tensor
from ttrl_amd.engine.nn import Module, ModuleList
from ttrl_amd.engine.ops import add, div, mean_dim, mul, relu, reshape, sqrt, square, sub, tanh
from ttrl_amd.engine.ops.fused import linear

__all__ = ["Linear", "LayerNorm", "ReLU", "Tanh", "Sequential", "Flatten"]


class Linear(Module):
    """y = x @ W + b, W stored (in_features, out_features)."""

    def __init__(self, in_features: int, out_features: int, device, *, bias: bool = True):
        if in_features <= 0 or out_features <= 0:
            raise ValueError(
                "Linear: in_features and out_features must be > 0, got "
                f"in_features={in_features}, out_features={out_features}"
            )
        self.in_features = int(in_features)
        self.out_features = int(out_features)
        bound = 1.0 / math.sqrt(in_features)
        weight = np.random.uniform(-bound, bound, (self.in_features, self.out_features)).astype(np.float32)
        self.weight = Tensor.from_numpy(weight, device, requires_grad=True)
        self.bias = None
        if bias:
            b = np.random.uniform(-bound, bound, (1, self.out_features)).astype(np.float32)
            self.bias = Tensor.from_numpy(b, device, requires_grad=True)

    def effective_weight(self):
        return self.weight

    def forward(self, x: Tensor) -> Tensor:
        return self.forward_fused(x, relu=False)

    def forward_fused(self, x: Tensor, relu: bool) -> Tensor:
        return linear(x, self.effective_weight(), self.bias, relu=relu)


class LayerNorm(Module):
    """(x - mean) / sqrt(var + eps) * gamma + beta over the last axis, composed."""

    def __init__(self, normalized_shape: int, device, *, eps: float = 1e-5):
        if normalized_shape <= 0:
            raise ValueError(f"LayerNorm: normalized_shape must be > 0, got {normalized_shape}")
        if eps <= 0.0:
            raise ValueError(
                f"LayerNorm: eps must be > 0, got {eps}; the variance of a "
                "constant row is zero and sqrt has no derivative there."
            )
        self.normalized_shape = int(normalized_shape)
        self.eps = float(eps)
        self.weight = Tensor.from_numpy(np.ones((1, self.normalized_shape), np.float32), device,
                                        requires_grad=True)
        self.bias = Tensor.from_numpy(np.zeros((1, self.normalized_shape), np.float32), device,
                                      requires_grad=True)

    def forward(self, x: Tensor) -> Tensor:
        if int(x.shape[-1]) != self.normalized_shape:
            raise ValueError(
                f"LayerNorm({self.normalized_shape}): expected a last axis of "
                f"{self.normalized_shape} features, got shape {tuple(int(d) for d in x.shape)}."
            )
        centred = sub(x, mean_dim(x, dim=-1))
        variance = mean_dim(square(centred), dim=-1)
        return add(mul(div(centred, sqrt(add(variance, self.eps))), self.weight), self.bias)


class ReLU(Module):
    """Elementwise max(x, 0)."""

    def forward(self, x: Tensor) -> Tensor:
        return relu(x)


class Tanh(Module):
    """Elementwise tanh(x)."""

    def forward(self, x: Tensor) -> Tensor:
        return tanh(x)


#: When set to a list, `Sequential.forward` appends the output array of every
#: fused layer+ReLU it runs (the device's gate pattern, for parity tests).
RECORD: list | None = None


def _fusable(layer) -> bool:
    return callable(getattr(layer, "forward_fused", None))


class Sequential(Module):
    """Chain layers; children are named `layers.<i>.<name>`."""

    def __init__(self, *layers):
        self.layers = ModuleList(layers)

    def forward(self, x: Tensor) -> Tensor:
        items = list(self.layers)
        i = 0
        while i < len(items):
            layer = items[i]
            if _fusable(layer) and i + 1 < len(items) and isinstance(items[i + 1], ReLU):
                x = layer.forward_fused(x, relu=True)
                if RECORD is not None:
                    RECORD.append(x.data)
                i += 2
                continue
            x = layer(x)
            i += 1
        return x

    def append(self, layer) -> "Sequential":
        self.layers.append(layer)
        return self

    def __len__(self) -> int:
        return len(self.layers)

    def __getitem__(self, index):
        return self.layers[index]


class Flatten(Module):
    """[1, 1, N*H*W, C] (flattened NHWC) -> (N, H*W*C), HWC feature order."""

    def __init__(self, h: int, w: int, channels: int):
        if h <= 0 or w <= 0 or channels <= 0:
            raise ValueError(f"Flatten: h, w and channels must be > 0, got {h}, {w}, {channels}")
        self.h = int(h)
        self.w = int(w)
        self.channels = int(channels)

    @property
    def out_features(self) -> int:
        return self.h * self.w * self.channels

    def forward(self, x: Tensor) -> Tensor:
        shape = tuple(int(d) for d in x.shape)
        rows = self.h * self.w
        if len(shape) != 4 or shape[0] != 1 or shape[1] != 1 or shape[3] != self.channels or shape[2] % rows != 0:
            raise ValueError(
                f"Flatten({self.h}, {self.w}, {self.channels}): expected "
                f"flattened-NHWC input of shape [1, 1, N*{self.h}*{self.w}, "
                f"{self.channels}], got {shape}"
            )
        return reshape(x, (shape[2] // rows, self.out_features))
