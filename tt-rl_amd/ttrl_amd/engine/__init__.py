"""ttrl_amd.engine: the MI355X compute substrate behind tt-rl's engine API
(ttrl/engine/__init__.py:15-92).  Importing it opens no device."""

from __future__ import annotations

import importlib
from typing import Any

from ttrl_amd.engine.config import DEFAULT, EngineConfig

_LAZY = {
    "Device": "device", "acquire": "device", "device_count": "device", "NoDeviceAvailable": "device",
    "DeviceProfile": "device", "open_device": "device", "purge_device_caches": "device",
    "register_device_cache": "device", "survey": "device", "probe_profile": "device",
    "DeviceArray": "tensor", "MASTER_DTYPE": "tensor", "ParamArena": "tensor", "copy_in_place": "tensor",
    "copy_tensor_in_place": "tensor", "to_device": "tensor", "to_host": "tensor", "restore_in_place": "tensor",
    "Tensor": "autograd", "backward": "autograd", "no_grad": "autograd",
    "Adam": "optim", "Optimizer": "optim", "adam_fused_scalars": "optim",
    "TrainStep": "step", "read_metrics": "step", "MODES": "step",
    "CapturedTrace": "trace", "TraceCaptureError": "trace", "capture": "trace",
    "Linear": "layers", "LayerNorm": "layers", "ReLU": "layers", "Tanh": "layers", "Sequential": "layers",
    "Flatten": "layers",
    "Conv2d": "conv", "ConvGeometry": "conv", "conv_out_size": "conv",
    "Module": "nn", "ModuleList": "nn", "ModuleDict": "nn",
}

_OPS = "ttrl_amd.engine.ops"

__all__ = ["DEFAULT", "EngineConfig", *sorted(_LAZY),
    "add", "div", "mul", "sub", "abs_", "exp", "log", "neg", "relu", "sigmoid", "sqrt", "square", "tanh",
    "clamp", "maximum", "minimum", "matmul", "argmax_dim_detached", "max_dim_detached", "mean_all", "mean_dim",
    "sum_all", "sum_dim", "concat", "reshape", "split", "apply_done_mask", "entropy", "gather_onehot", "huber",
    "log_softmax", "masks", "non_finite_check", "one_hot_device", "one_hot_gather", "one_hot_host",
    "linear", "dqn_td_loss",
]


def __getattr__(name: str) -> Any:
    module = _LAZY.get(name)
    if module is not None:
        return getattr(importlib.import_module(f"ttrl_amd.engine.{module}"), name)
    if name in __all__:
        return getattr(importlib.import_module(_OPS), name)
    raise AttributeError(f"module {__name__!r} has no attribute {name!r}")


def __dir__() -> list[str]:
    return sorted(__all__)
