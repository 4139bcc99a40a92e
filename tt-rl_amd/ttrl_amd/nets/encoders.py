"""Observation encoders (ttrl/nets/encoders.py:50-237).

`image_encoder`: Conv2d+ReLU per tower stage, Flatten (HWC order),
Linear(hidden)+ReLU; the first stage folds `ObsSpec.scale` and has no input
gradient.  A uint8 image spec makes the first stage read the frames as they
come from the environment (uint8 NCHW), so no host-side layout conversion or
float cast is needed before upload.
`vector_encoder`: ScaledLinear+ReLU per hidden width.
`identity_encoder`: the raw vector row (the SAC critic's fusion point).
"""

from __future__ import annotations

from ttrl_amd.engine.conv import Conv2d
from ttrl_amd.engine.layers import Flatten, Linear, ReLU, Sequential
from ttrl_amd.engine.ops import mul
from ttrl_amd.nets.towers import NATURE_CNN


class ScaledLinear(Linear):
    """y = (scale * x) @ W + b with the scale folded into the weight."""

    def __init__(self, in_features: int, out_features: int, device, *, scale: float = 1.0, bias: bool = True):
        super().__init__(in_features, out_features, device, bias=bias)
        if not scale > 0.0:
            raise ValueError(f"ScaledLinear: scale must be positive, got {scale}")
        self.scale = float(scale)

    def effective_weight(self):
        return self.weight if self.scale == 1.0 else mul(self.weight, self.scale)


class Encoder(Sequential):
    """A Sequential that reports the width of the row it emits."""

    def __init__(self, layers, out_features: int):
        super().__init__(*layers)
        self.out_features = int(out_features)


def image_encoder(obs_spec, device, *, batch: int, hidden: int = 512, tower=NATURE_CNN,
                  input_needs_grad: bool = False) -> Encoder:
    if obs_spec.kind != "image":
        raise ValueError(
            f"image encoder needs an image ObsSpec, got kind={obs_spec.kind!r} with "
            f"shape {obs_spec.shape}. A vector observation has no spatial geometry; use the 'mlp' encoder."
        )
    if hidden < 1:
        raise ValueError(f"image encoder: hidden must be >= 1, got {hidden}")
    if not tower:
        raise ValueError("image encoder: tower must hold at least one ConvStage")
    in_shape = obs_spec.shape
    layers = []
    for index, stage in enumerate(tower):
        first = index == 0
        layout = "nchw_u8" if first and obs_spec.dtype == "uint8" else "nhwc"
        conv = Conv2d(in_shape, stage.out_channels, stage.kernel, device, batch=batch, stride=stage.stride,
                      padding=stage.padding, input_scale=obs_spec.scale if first else 1.0,
                      needs_input_grad=input_needs_grad if first else True, input_layout=layout)
        layers += [conv, ReLU()]
        in_shape = conv.out_shape
    channels, height, width = in_shape
    flatten = Flatten(height, width, channels)
    layers += [flatten, Linear(flatten.out_features, hidden, device), ReLU()]
    return Encoder(layers, hidden)


def vector_encoder(obs_spec, device, *, batch: int = 0, hidden=(256, 256)) -> Encoder:
    if obs_spec.kind != "vector":
        raise ValueError(
            f"mlp encoder needs a vector ObsSpec, got kind={obs_spec.kind!r} with shape {obs_spec.shape}. "
            "Use the 'nature_cnn' encoder for images."
        )
    widths = tuple(int(w) for w in hidden)
    if not widths or min(widths) < 1:
        raise ValueError(f"mlp encoder: hidden must be positive widths, got {hidden}")
    layers = []
    in_features = obs_spec.size
    for index, width in enumerate(widths):
        layers += [ScaledLinear(in_features, width, device, scale=obs_spec.scale if index == 0 else 1.0), ReLU()]
        in_features = width
    return Encoder(layers, widths[-1])


def identity_encoder(obs_spec, device, *, batch: int = 0) -> Encoder:
    if obs_spec.kind != "vector":
        raise ValueError(
            f"identity encoder needs a vector ObsSpec, got kind={obs_spec.kind!r} with shape {obs_spec.shape}."
        )
    if obs_spec.scale != 1.0:
        raise ValueError(
            f"identity encoder: this leaf declares scale={obs_spec.scale}, and a tower of no layers has no "
            "weight to fold it into."
        )
    return Encoder((), obs_spec.size)
