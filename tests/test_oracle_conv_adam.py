"""Pins of the oracle's convolution, geometry and Adam.

Known answers are the reference's own (tests/engine/test_geometry_and_scalars.py:16-50,
ttrl/nets/towers.py:37-40, the Nature-CNN parameter count); the convolution is
checked against brute-force loops, adjointness <conv(x), y> = <x, conv^T(y)>
and torch's float64 conv2d with autograd (an independent implementation)."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import adam, conv


@pytest.mark.parametrize("size, kernel, stride, padding, expected", [(84, 8, 4, 0, 20), (5, 3, 1, 1, 5)])
def test_conv_out_size_known_answers(size, kernel, stride, padding, expected):
    from ttrl_amd.engine.conv import conv_out_size
    assert conv.out_size(size, kernel, stride, padding) == expected
    assert conv_out_size(size, kernel, stride, padding) == expected


def test_ragged_geometry_is_refused():
    from ttrl_amd.engine.conv import conv_out_size
    with pytest.raises(ValueError):
        conv.out_size(6, 3, 2, 0)
    with pytest.raises(ValueError, match="ragged"):
        conv_out_size(6, 3, 2, 0)


def test_nature_cnn_geometry_and_parameter_count():
    h = 84
    for k, s in ((8, 4), (4, 2), (3, 1)):
        h = conv.out_size(h, k, s)
    assert h == 7 and 7 * 7 * 64 == 3136
    params = (32 * 4 * 64 + 32) + (64 * 32 * 16 + 64) + (64 * 64 * 9 + 64) + (3136 * 512 + 512) + (512 * 6 + 6)
    assert params == 1_687_206


def _brute(x, w, b, s, p):
    n, h, wd, c = x.shape
    o, _, k, _ = w.shape
    xp = np.pad(x, ((0, 0), (p, p), (p, p), (0, 0)))
    oh, ow = (h + 2 * p - k) // s + 1, (wd + 2 * p - k) // s + 1
    y = np.zeros((n, oh, ow, o))
    for a in range(n):
        for i in range(oh):
            for j in range(ow):
                for q in range(o):
                    acc = b[q]
                    for cc in range(c):
                        for u in range(k):
                            for v in range(k):
                                acc += xp[a, i * s + u, j * s + v, cc] * w[q, cc, u, v]
                    y[a, i, j, q] = acc
    return y


@pytest.mark.parametrize("c,o,k,s,p,h", [(2, 3, 3, 1, 0, 5), (3, 2, 4, 2, 0, 8), (2, 2, 3, 2, 1, 7)])
def test_conv_forward_brute_force(c, o, k, s, p, h):
    rng = np.random.default_rng(c * 100 + o * 10 + k)
    x = rng.standard_normal((2, h, h, c))
    w = rng.standard_normal((o, c, k, k))
    b = rng.standard_normal(o)
    np.testing.assert_allclose(conv.forward(x, w, b, s, p), _brute(x, w, b, s, p), rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("c,o,k,s,p,h", [(4, 8, 8, 4, 0, 36), (8, 6, 4, 2, 0, 12), (5, 4, 3, 1, 1, 9),
                                         (3, 5, 3, 2, 1, 11)])
def test_conv_backward_adjoint_and_torch(c, o, k, s, p, h):
    rng = np.random.default_rng(k * 7 + s)
    x = rng.standard_normal((3, h, h, c))
    w = rng.standard_normal((o, c, k, k))
    b = rng.standard_normal(o)
    y = conv.forward(x, w, b, s, p)
    dy = rng.standard_normal(y.shape)
    dx, dw, db = conv.backward(x, w, dy, s, p)
    # adjointness of the linear map x -> conv(x, w) (no bias)
    lhs = np.sum((conv.forward(x, w, None, s, p)) * dy)
    assert math.isclose(lhs, np.sum(x * dx), rel_tol=1e-10)
    # independent implementation: torch float64 conv2d + autograd (NCHW)
    xt = torch.tensor(x.transpose(0, 3, 1, 2), requires_grad=True)
    wt = torch.tensor(w, requires_grad=True)
    bt = torch.tensor(b, requires_grad=True)
    yt = torch.nn.functional.conv2d(xt, wt, bt, stride=s, padding=p)
    np.testing.assert_allclose(yt.detach().numpy().transpose(0, 2, 3, 1), y, rtol=1e-10, atol=1e-10)
    yt.backward(torch.tensor(dy.transpose(0, 3, 1, 2)))
    np.testing.assert_allclose(xt.grad.numpy().transpose(0, 2, 3, 1), dx, rtol=1e-10, atol=1e-10)
    np.testing.assert_allclose(wt.grad.numpy(), dw, rtol=1e-10, atol=1e-10)
    np.testing.assert_allclose(bt.grad.numpy(), db, rtol=1e-10, atol=1e-10)


@pytest.mark.parametrize("t", [1, 10, 100_000])
def test_fused_scalars_reproduce_textbook_adam(t):
    """The reference's known answer (tests/engine/test_geometry_and_scalars.py:40-50)."""
    from ttrl_amd.engine.optim import adam_fused_scalars
    lr, b1, b2, eps = 1e-4, 0.9, 0.999, 1e-8
    m, v = 0.37, 0.0021
    S, V = m / (1 - b1), v / (1 - b2)
    want = lr * (m / (1 - b1 ** t)) / (math.sqrt(v / (1 - b2 ** t)) + eps)
    for fn in (adam.fused_scalars, adam_fused_scalars):
        alpha_t, eps_t = fn(lr, b1, b2, eps, t)
        assert alpha_t * S / (math.sqrt(V) + eps_t) == pytest.approx(want, rel=1e-12)


def test_fused_adam_equals_textbook_and_torch_over_steps():
    rng = np.random.default_rng(0)
    p0 = rng.uniform(-1, 1, 64)
    pf, S, V = p0.copy(), np.zeros(64), np.zeros(64)
    pt, m, v = p0.copy(), np.zeros(64), np.zeros(64)
    tp = torch.tensor(p0.copy(), requires_grad=True)
    opt = torch.optim.Adam([tp], lr=1e-3, eps=1e-8)
    for t in range(1, 8):
        g = rng.uniform(-0.1, 0.1, 64)
        pf, S, V = adam.fused_step(pf, g, S, V, t, 1e-3)
        pt, m, v = adam.textbook_step(pt, g, m, v, t, 1e-3)
        tp.grad = torch.tensor(g)
        opt.step()
        np.testing.assert_allclose(pf, pt, rtol=1e-12, atol=1e-14)
        np.testing.assert_allclose(pf, tp.detach().numpy(), rtol=1e-12, atol=1e-14)
    # canonical m, v from the stored form (ttrl/engine/optim/checkpoint.py:15-27)
    np.testing.assert_allclose(S * (1 - 0.9), m, rtol=1e-12)
    np.testing.assert_allclose(V * (1 - 0.999), v, rtol=1e-12)


def test_adam_step_one_closed_form():
    """At t = 1 from zero state: p1 = p0 - lr * g / (|g| + eps) exactly."""
    rng = np.random.default_rng(1)
    p0, g = rng.standard_normal(50), rng.standard_normal(50) * 1e-3
    p1, _, _ = adam.fused_step(p0, g, np.zeros(50), np.zeros(50), 1, 6.25e-5, eps=1.5e-4)
    np.testing.assert_allclose(p1, p0 - 6.25e-5 * g / (np.abs(g) + 1.5e-4), rtol=1e-12)


def test_planted_mistake_in_conv_is_caught():
    """A transposed kernel (a plausible indexing slip) must fail the torch pin."""
    rng = np.random.default_rng(3)
    x = rng.standard_normal((1, 9, 9, 2))
    w = rng.standard_normal((3, 2, 3, 3))
    wrong = conv.forward(x, w.transpose(0, 1, 3, 2), None, 1, 0)
    yt = torch.nn.functional.conv2d(torch.tensor(x.transpose(0, 3, 1, 2)), torch.tensor(w))
    assert not np.allclose(wrong, yt.numpy().transpose(0, 2, 3, 1))
