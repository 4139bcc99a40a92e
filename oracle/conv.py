"""Convolution in float64 on NHWC arrays, restated from the reference.

forward   ttrl/deploy/conv.py:31-50 (sliding-window im2col, patch order (c, kh, kw))
dW, db    ttrl/engine/conv/backward.py:45-78 (dW[k,c,p,q] = sum dY[n,i,j,k] X[n,i*s+p,j*s+q,c])
dX        ttrl/engine/conv/backward.py:33-42 (the adjoint of the forward)
"""

from __future__ import annotations

import numpy as np

from oracle import fa, float_type


def out_size(size: int, kernel: int, stride: int, padding: int = 0) -> int:
    """(size + 2p - k)/s + 1, refusing ragged geometry (ttrl/engine/conv/geometry.py:107-119)."""
    span = size + 2 * padding - kernel
    if span < 0 or span % stride:
        raise ValueError(f"ragged geometry: size {size}, kernel {kernel}, stride {stride}, padding {padding}")
    return span // stride + 1


def _windows(x: np.ndarray, k: int, s: int, p: int) -> np.ndarray:
    """(N, OH, OW, C, k, k) windows of padded NHWC x."""
    if p:
        x = np.pad(x, ((0, 0), (p, p), (p, p), (0, 0)))
    return np.lib.stride_tricks.sliding_window_view(x, (k, k), axis=(1, 2))[:, ::s, ::s]


def forward(x: np.ndarray, w: np.ndarray, b: np.ndarray | None, stride: int, padding: int = 0) -> np.ndarray:
    """y[n,i,j,o] = sum_{c,p,q} x[n, i*s+p, j*s+q, c] w[o,c,p,q] + b[o]; x NHWC, w OIHW."""
    x = fa(x)
    w = fa(w)
    o, _, k, _ = w.shape
    win = _windows(x, k, stride, padding)
    n, oh, ow = win.shape[:3]
    cols = win.reshape(n * oh * ow, -1)
    y = cols @ w.reshape(o, -1).T
    if b is not None:
        y = y + fa(b).reshape(-1)
    return y.reshape(n, oh, ow, o)


def backward(x: np.ndarray, w: np.ndarray, dy: np.ndarray, stride: int, padding: int = 0,
             need_dx: bool = True):
    """(dx NHWC | None, dw OIHW, db (O,)) for y = forward(x, w, b)."""
    x = fa(x)
    w = fa(w)
    dy = fa(dy)
    o, c, k, _ = w.shape
    win = _windows(x, k, stride, padding)  # (n, oh, ow, c, k, k)
    dw = np.einsum("nijckl,nijo->ockl", win, dy, optimize=True)
    db = dy.sum(axis=(0, 1, 2))
    dx = None
    if need_dx:
        n, h, wd, _ = x.shape
        oh, ow = dy.shape[1], dy.shape[2]
        dxp = np.zeros((n, h + 2 * padding, wd + 2 * padding, c), float_type())
        # contribution of every output pixel to its input window
        contrib = np.einsum("nijo,ockl->nijklc", dy, w, optimize=True)
        for p in range(k):
            for q in range(k):
                dxp[:, p:p + stride * (oh - 1) + 1:stride, q:q + stride * (ow - 1) + 1:stride, :] += contrib[:, :, :, p, q, :]
        dx = dxp[:, padding:padding + h, padding:padding + wd, :]
    return dx, dw, db
