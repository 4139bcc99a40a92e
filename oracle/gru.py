"""Float64 restatement of the GRU unroll (ttrl/engine/recurrent.py:39-168).

Test infrastructure only.  Cell (PyTorch's gate order and placement of the
reset gate; weights stored (in, 3 * hidden), stacked reset | update |
candidate):

    gi = x W_ih + b_ih, gh = h W_hh + b_hh
    r = sigmoid(gi_r + gh_r), z = sigmoid(gi_z + gh_z)
    n = tanh(gi_n + r * gh_n), h' = (1 - z) * n + z * h

Unroll: the state entering step t is h_{t-1} * (1 - done_t)
(apply_done_mask, ttrl/engine/ops/functional.py:40-46); the outputs are the
states after every step.  The backward is the analytic reverse of the same
composition.
"""

from __future__ import annotations

import numpy as np


def _sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


def gru_forward(W_ih, W_hh, b_ih, b_hh, x, h0, done=None):
    """-> (outputs (T, B, H), cache)."""
    x = np.asarray(x, np.float64)
    T, B, _ = x.shape
    H = W_hh.shape[0]
    keep = np.ones((T, B, 1)) if done is None else 1.0 - np.asarray(done, np.float64).reshape(T, B, 1)
    h = np.asarray(h0, np.float64)
    outs, cache = [], []
    for t in range(T):
        hin = h * keep[t]
        gi = x[t] @ W_ih + b_ih.reshape(1, -1)
        gh = hin @ W_hh + b_hh.reshape(1, -1)
        r = _sigmoid(gi[:, :H] + gh[:, :H])
        z = _sigmoid(gi[:, H:2 * H] + gh[:, H:2 * H])
        n = np.tanh(gi[:, 2 * H:] + r * gh[:, 2 * H:])
        h = (1.0 - z) * n + z * hin
        outs.append(h)
        cache.append((hin, gh, r, z, n))
    return np.stack(outs), (x, keep, cache, W_ih, W_hh)


def gru_backward(cache, dout):
    """-> (dx, dh0, dW_ih, dW_hh, db_ih, db_hh) for upstream d outputs."""
    x, keep, steps, W_ih, W_hh = cache
    T, B, F = x.shape
    H = W_hh.shape[0]
    dx = np.zeros_like(x)
    dW_ih, dW_hh = np.zeros_like(W_ih, dtype=np.float64), np.zeros_like(W_hh, dtype=np.float64)
    db_ih, db_hh = np.zeros(3 * H), np.zeros(3 * H)
    dh_next = np.zeros((B, H))  # gradient w.r.t. the output state of step t from later steps
    for t in range(T - 1, -1, -1):
        hin, gh, r, z, n = steps[t]
        dh = np.asarray(dout[t], np.float64) + dh_next
        dn = dh * (1.0 - z)
        dz = dh * (hin - n)
        dhin = dh * z
        dnp = dn * (1.0 - n * n)
        dr = dnp * gh[:, 2 * H:]
        drp = dr * r * (1.0 - r)
        dzp = dz * z * (1.0 - z)
        dgi = np.concatenate([drp, dzp, dnp], axis=1)
        dgh = np.concatenate([drp, dzp, dnp * r], axis=1)
        dW_ih += x[t].T @ dgi
        db_ih += dgi.sum(axis=0)
        dW_hh += hin.T @ dgh
        db_hh += dgh.sum(axis=0)
        dx[t] = dgi @ W_ih.T
        dhin = dhin + dgh @ W_hh.T
        dh_next = dhin * keep[t]
    return dx, dh_next, dW_ih, dW_hh, db_ih, db_hh
