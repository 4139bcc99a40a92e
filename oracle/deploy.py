"""Test infrastructure only (imported by tests/): the reference's deployed
policy forward restated in float64 numpy, read straight off an artifact
file, to check what `ttrl_amd.deploy` writes and runs.

Follows ttrl/deploy/artifact.py:188-203 and 238-252 (raw observation as float, conv
stages, trunk Linear + ReLU, head, action map) and ttrl/deploy/conv.py:31-50
(each conv stage as one matmul over strided NHWC windows, OIHW weights
flattened in (C, kh, kw) order, ReLU, NHWC flatten).  Pinned in
tests/test_deploy.py: the conv path against oracle/nets.qnet_forward (itself
pinned against torch's conv2d) on the same weights, and the action maps
against their closed forms.
"""

from __future__ import annotations

import json

import numpy as np

from oracle import fa, float_type

__all__ = ["read", "head_rows", "actions"]


def read(path: str) -> tuple[dict, dict]:
    with np.load(path, allow_pickle=False) as npz:
        meta = json.loads(npz["__meta__"].tobytes().decode("utf-8"))
        arrays = {k: npz[k] for k in npz.files if k != "__meta__"}
    return meta, arrays


def _conv_features(rows: np.ndarray, stages: list) -> np.ndarray:
    """(batch, C, H, W) -> (batch, features), NHWC flatten (ttrl/deploy/conv.py:31-50)."""
    hidden = np.ascontiguousarray(rows.transpose(0, 2, 3, 1))
    for weight, bias, stride, padding in stages:
        out_channels, _, kernel, _ = weight.shape
        if padding:
            hidden = np.pad(hidden, ((0, 0), (padding, padding), (padding, padding), (0, 0)))
        windows = np.lib.stride_tricks.sliding_window_view(hidden, (kernel, kernel), axis=(1, 2))[:, ::stride, ::stride]
        batch, height, width = windows.shape[:3]
        columns = windows.reshape(batch * height * width, -1)  # (C, kh, kw) order
        out = columns @ weight.reshape(out_channels, -1).T + bias
        hidden = np.maximum(out, 0.0).reshape(batch, height, width, out_channels)
    return hidden.reshape(hidden.shape[0], -1)


def head_rows(meta: dict, arrays: dict, obs: np.ndarray) -> np.ndarray:
    """The head's raw rows for a batch of raw observations
    (ttrl/deploy/artifact.py:188-203, ttrl/deploy/conv.py:22-29)."""
    shape = tuple(int(d) for d in meta["obs_shape"])
    hidden = fa(obs).reshape((-1,) + shape)
    if meta["conv"]:
        stages = [(arrays[f"conv.{i}.weight"].astype(float_type(), copy=False), arrays[f"conv.{i}.bias"].astype(float_type(), copy=False),
                   int(g["stride"]), int(g["padding"])) for i, g in enumerate(meta["conv"])]
        hidden = _conv_features(hidden, stages)
    for i in range(int(meta["trunk_layers"])):
        hidden = np.maximum(hidden @ arrays[f"trunk.{i}.weight"].astype(float_type(), copy=False)
                            + arrays[f"trunk.{i}.bias"].astype(float_type(), copy=False), 0.0)
    return hidden @ arrays["head.weight"].astype(float_type(), copy=False) + arrays["head.bias"].astype(float_type(), copy=False)


def actions(meta: dict, arrays: dict, obs: np.ndarray) -> np.ndarray:
    """The deterministic actions (ttrl/deploy/artifact.py:238-252): the first
    argmax, centre + half_width * tanh(mean), or mean clipped to the bounds."""
    row = head_rows(meta, arrays, obs)
    kind = meta["action_map"]
    if kind == "argmax":
        return np.argmax(row, axis=-1).astype(np.int64)
    low = arrays["action_low"].astype(float_type(), copy=False)
    high = arrays["action_high"].astype(float_type(), copy=False)
    if kind == "tanh_bounds":
        return (high + low) * 0.5 + (high - low) * 0.5 * np.tanh(row)
    if kind == "clip_bounds":
        return np.clip(row, low, high)
    raise ValueError(f"unknown action map {kind!r}")
