"""Gradients and parameter deltas of a module, in its state_dict layout.

`grad_state(module)` reads every parameter's current gradient (the arena
gradient slot an update wrote) and returns it under the parameter's
state_dict key, conv weights converted to logical OIHW like the weights
themselves, so it lines up with the oracle's per-parameter lists."""

from __future__ import annotations

import numpy as np


def grad_of(p) -> np.ndarray:
    g = p.grad if p.grad is not None else p._grad_slot
    if g is None:
        raise AssertionError("parameter has no gradient buffer")
    return g.numpy().reshape(tuple(p.shape))


def grad_state(module) -> dict:
    from ttrl_amd.engine.autograd import Tensor
    from ttrl_amd.engine.conv import Conv2d, master_to_oihw

    out = {}
    for name, target in module._state_slots():
        if isinstance(target, Tensor):
            out[name] = grad_of(target)
        elif isinstance(target, Conv2d):
            g = grad_of(target.weight)
            out[f"{name}.weight"] = master_to_oihw(g, target._oihw_shape, target.input_layout)
            if target.bias is not None:
                out[f"{name}.bias"] = grad_of(target.bias)
        else:
            raise AssertionError(f"grad_state: no gradient reader for {type(target).__name__} at {name}")
    return out


def rel_err(got, ref) -> float:
    """max |got - ref| over the tensor relative to max |ref|."""
    ref = np.asarray(ref, np.float64)
    got = np.asarray(got, np.float64).reshape(ref.shape)
    return float(np.max(np.abs(got - ref)) / max(np.max(np.abs(ref)), 1e-30))


def check_grads(got: dict, want: list, rel: float, label: str = "") -> None:
    """Each gradient tensor within `rel` of its own scale (max |g|)."""
    assert len(got) == len(want), (label, len(got), len(want))
    for (k, g), w in zip(got.items(), want):
        err = rel_err(g, w)
        assert err < rel, (label, k, err)


def check_deltas(p0: list, p1: list, want1: list, rel: float, label: str = "", skip=None) -> int:
    """Adam deltas p1 - p0 against the oracle's want1 - p0, within `rel` of
    the largest oracle delta of the tensor plus the float32 spacing of the
    parameter (a float32 parameter resolves its delta to one ulp).  `skip`
    (optional list of boolean masks) excludes entries from the comparison;
    returns how many were excluded."""
    skipped = 0
    for i, (a, b, w) in enumerate(zip(p0, p1, want1)):
        w = np.asarray(w, np.float64)
        a = np.asarray(a, np.float64).reshape(w.shape)
        b = np.asarray(b, np.float64).reshape(w.shape)
        d, dw = b - a, w - a
        ulp = np.spacing(np.maximum(np.abs(a), np.abs(b)).astype(np.float32)).astype(np.float64)
        tol = rel * np.max(np.abs(dw)) + ulp
        ok = np.abs(d - dw) <= tol
        if skip is not None:
            m = np.asarray(skip[i]).reshape(w.shape)
            skipped += int(m.sum())
            ok |= m
        assert np.all(ok), (label, i, float(np.max(np.abs(d - dw) / np.maximum(tol, 1e-30))))
    return skipped
