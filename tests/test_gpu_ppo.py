"""PPO kernels on the GPU against the oracle: the GAE scan bit-exact against
the oracle's float32 recursion (same rounding as the reference), the
advantage normalisation, the fused objective and its gradients (fp32 vs
float64, rel 1e-4 of each quantity's scale), the tape node's backward, and
the device global-norm clip."""

from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from oracle import ppo as oppo
from ttrl_amd import _lib

pytestmark = pytest.mark.gpu


def _rel(got, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


def _rollout(seed, T, N, padded):
    rng = np.random.default_rng(seed)
    r = rng.choice([-1.0, 0.0, 1.0], (T, N), p=[0.05, 0.9, 0.05]).astype(np.float32)
    v = rng.normal(size=(T, N)).astype(np.float32)
    d = (rng.random((T, N)) < 0.01).astype(np.float32)
    last = rng.normal(size=N).astype(np.float32)
    valid = (rng.random((T, N)) > 0.05).astype(np.float32) if padded else None
    return r, v, d, last, valid


@pytest.mark.parametrize("T,N,padded", [(128, 8, False), (128, 8, True), (100, 70, True), (1, 1, False),
                                        (200, 3, False)])
def test_gae_bit_exact(device, T, N, padded):
    from ttrl_amd.algos.ppo import compute_gae
    r, v, d, last, valid = _rollout(T * 1000 + N, T, N, padded)
    adv, ret = compute_gae(device, r, v, d, last, 0.99, 0.95, valid)
    adv_ref, ret_ref = oppo.gae(r, v, d, last, 0.99, 0.95, valid)
    assert np.array_equal(adv.numpy(), adv_ref)
    assert np.array_equal(ret.numpy(), ret_ref)


def test_normalize_advantages(device):
    from ttrl_amd.algos.ppo import normalize_advantages
    rng = np.random.default_rng(3)
    a = rng.normal(2.0, 3.0, (128, 8)).astype(np.float32)
    valid = (rng.random((128, 8)) > 0.1).astype(np.float32)
    for w in (None, valid):
        out, stats = normalize_advantages(device, a, w)
        ref, mean, std = oppo.normalize_advantages(a, w)
        assert _rel(out.numpy(), ref) < 1e-5
        assert abs(stats.numpy()[0] - mean) < 1e-5 * abs(mean) and abs(stats.numpy()[1] - std) < 1e-5 * std


def _minibatch(seed, B, A):
    rng = np.random.default_rng(seed)
    z = rng.normal(size=(B, A)).astype(np.float32)
    a = rng.integers(0, A, B)
    old_lp = (oppo.log_softmax(z)[np.arange(B), a] + rng.normal(0, 0.15, B)).astype(np.float32)
    adv = rng.normal(size=B).astype(np.float32)
    ret = rng.normal(size=B).astype(np.float32)
    old_v = rng.normal(size=B).astype(np.float32)
    v = (old_v + rng.normal(0, 0.2, B)).astype(np.float32)
    return z, a, old_lp, adv, ret, old_v, v


@pytest.mark.parametrize("masked", [False, True])
@pytest.mark.parametrize("B,A", [(256, 18), (300, 6), (1500, 32), (200, 40)])
def test_ppo_loss_matches_oracle(device, masked, B, A):
    """Up to 32 actions the rows sit in registers (several rows per thread
    past 1024); more actions take the general kernel."""
    from ttrl_amd.engine.tensor import DeviceArray, to_device
    z, a, old_lp, adv, ret, old_v, v = _minibatch(11 + masked, B, A)
    w = (np.random.default_rng(2).random(B) > 0.3).astype(np.float32) if masked else None
    cfg = dict(clip_eps=0.1, value_clip_eps=0.1, value_coef=0.5, entropy_coef=0.01)
    d = {k: to_device(x, device) for k, x in (("z", z), ("old_lp", old_lp), ("adv", adv), ("ret", ret),
                                                ("old_v", old_v), ("v", v))}
    ad = to_device(a.astype(np.int32), device, np.int32)
    wd = None if w is None else to_device(w, device)
    out4 = DeviceArray(device, (4,))
    nlp, dz, dv = DeviceArray(device, (B,)), DeviceArray(device, (B, A)), DeviceArray(device, (B,))
    device.call("ttrl_ppo_loss", B, A, d["z"].vp, ad.vp, d["old_lp"].vp, d["adv"].vp, d["ret"].vp, d["old_v"].vp,
                d["v"].vp, None if wd is None else wd.vp, C.c_float(0.1), C.c_float(0.1), C.c_float(0.5),
                C.c_float(0.01), out4.vp, nlp.vp, dz.vp, dv.vp)
    ref = oppo.ppo_objective(z, a, old_lp, adv, ret, old_v, v, w, **cfg)
    got = out4.numpy()
    for i, key in enumerate(("loss", "policy_loss", "value_loss", "entropy")):
        assert abs(got[i] - ref[key]) < 1e-4 * max(abs(ref[key]), 1e-3), key
    assert _rel(nlp.numpy(), ref["new_logp"]) < 1e-5
    assert _rel(dz.numpy(), ref["dlogits"]) < 1e-4
    assert _rel(dv.numpy(), ref["dvalues"]) < 1e-4


def test_ppo_objective_tape_node(device):
    from ttrl_amd.algos.ppo import PPOLossConfig, objective
    from ttrl_amd.engine.autograd import Tensor
    B, A = 64, 18
    z, a, old_lp, adv, ret, old_v, v = _minibatch(21, B, A)
    logits = Tensor.from_numpy(z, device, requires_grad=True)
    value = Tensor.from_numpy(v.reshape(B, 1), device, requires_grad=True)
    batch = dict(actions=a, old_logp=old_lp, advantages=adv, returns=ret, values=old_v)
    loss, parts, new_logp = objective(logits, value, batch, PPOLossConfig())
    loss.backward()
    ref = oppo.ppo_objective(z, a, old_lp, adv, ret, old_v, v, clip_eps=0.1, value_clip_eps=0.1, value_coef=0.5,
                             entropy_coef=0.01)
    assert abs(loss.numpy().reshape(-1)[0] - ref["loss"]) < 1e-4 * abs(ref["loss"])
    assert _rel(logits.grad.numpy(), ref["dlogits"]) < 1e-4
    assert _rel(value.grad.numpy().reshape(-1), ref["dvalues"]) < 1e-4
    assert _rel(new_logp.numpy().reshape(-1), ref["new_logp"]) < 1e-5


@pytest.mark.parametrize("max_norm", [0.5, 1e6])
def test_clip_grad_norm_device(device, max_norm):
    from ttrl_amd.algos.ppo import clip_grad_norm_device
    from ttrl_amd.engine.tensor import to_device
    g = np.random.default_rng(5).normal(0, 0.01, 1_687_206).astype(np.float32)
    gd = to_device(g, device)
    norm = clip_grad_norm_device(gd, max_norm)
    ref, ref_norm = oppo.clip_grad_norm(g, max_norm)
    assert abs(norm.numpy()[0] - ref_norm) < 1e-5 * ref_norm
    assert _rel(gd.numpy(), ref) < 1e-6


@pytest.mark.parametrize("n,max_norm", [(1_687_206, 0.5), (1_687_206, 1e6), (10_007, 0.05)])
def test_clipped_adam_step_is_the_clip_then_the_step(device, n, max_norm):
    """ttrl_adam_step_clipped against ttrl_clip_grad_norm followed by
    ttrl_adam_step, bit for bit: parameters, moments, the gradient left in
    place, the norm, the sum of squares and the update count, over two
    steps (a ragged tail, clipping on and off)."""
    from ttrl_amd.engine.tensor import DeviceArray, to_device

    rng = np.random.default_rng(n)
    p0 = rng.uniform(-1, 1, n).astype(np.float32)
    g0 = rng.normal(0, 0.01, n).astype(np.float32)
    runs = []
    for fused in (False, True):
        p, g = to_device(p0, device), to_device(g0, device)
        S, V = DeviceArray(device, (n,)), DeviceArray(device, (n,))
        S.fill(0.0)
        V.fill(0.0)
        step = to_device(np.zeros(1, np.int32), device, np.int32)
        sq, norm, gsq = DeviceArray(device, (1,)), DeviceArray(device, (1,)), DeviceArray(device, (1,))
        hyper = (C.c_float(2.5e-4), C.c_float(0.9), C.c_float(0.999), C.c_float(1e-5), C.c_float(0.0))
        for _ in range(2):
            if fused:
                device.call("ttrl_adam_step_clipped", p.vp, g.vp, S.vp, V.vp, C.c_long(n), step.vp, *hyper, gsq.vp, 0,
                            C.c_float(max_norm), sq.vp, norm.vp)
            else:
                device.call("ttrl_clip_grad_norm", g.vp, C.c_long(n), C.c_float(max_norm), sq.vp, norm.vp)
                device.call("ttrl_adam_step", p.vp, g.vp, S.vp, V.vp, C.c_long(n), step.vp, *hyper, gsq.vp, 0)
        runs.append([x.numpy() for x in (p, g, S, V, sq, norm, gsq)] + [step.numpy()])
    for name, a, b in zip(("p", "g", "S", "V", "sq", "norm", "grad_sq", "step"), *runs):
        assert np.array_equal(a, b), name
    assert runs[1][-1][0] == 2


def test_clipped_adam_step_with_the_step_end_is_the_two_calls(device):
    """ttrl_adam_step_clipped_end against ttrl_adam_step_clipped followed by
    ttrl_step_end, bit for bit: parameters, moments, gradient, norm, sums of
    squares, update count, metric ring and step counter, over three steps
    whose metrics hold the step's own norm (the PPO learner's layout) and
    whose last one finds the ring full (the counter still advances)."""
    from ttrl_amd.engine.tensor import DeviceArray, to_device

    n, n_metrics, slots = 70001, 7, 2
    rng = np.random.default_rng(3)
    p0 = rng.uniform(-1, 1, n).astype(np.float32)
    g0 = rng.normal(0, 0.01, n).astype(np.float32)
    m0 = rng.normal(0, 1, n_metrics).astype(np.float32)
    runs = []
    for fused in (False, True):
        p, g = to_device(p0, device), to_device(g0, device)
        S, V = DeviceArray(device, (n,)), DeviceArray(device, (n,))
        S.fill(0.0)
        V.fill(0.0)
        step = to_device(np.zeros(1, np.int32), device, np.int32)
        counter = to_device(np.zeros(1, np.int32), device, np.int32)
        metrics = to_device(m0, device)
        ring = to_device(np.full((slots, n_metrics), -1.0, np.float32), device)
        sq, gsq = DeviceArray(device, (1,)), DeviceArray(device, (1,))
        norm = C.c_void_p(metrics.ptr + 4 * 5)
        hyper = (C.c_float(2.5e-4), C.c_float(0.9), C.c_float(0.999), C.c_float(1e-5), C.c_float(0.0))
        for k in range(3):
            args = (p.vp, g.vp, S.vp, V.vp, C.c_long(n), step.vp, *hyper, gsq.vp, 0, C.c_float(0.5 if k else 1e-3),
                    sq.vp, norm)
            if fused:
                device.call("ttrl_adam_step_clipped_end", *args, counter.vp, metrics.vp, n_metrics, ring.vp, slots)
            else:
                device.call("ttrl_adam_step_clipped", *args)
                device.call("ttrl_step_end", counter.vp, metrics.vp, n_metrics, ring.vp, slots)
        runs.append([x.numpy() for x in (p, g, S, V, sq, gsq, metrics, ring, step, counter)])
    for name, a, b in zip(("p", "g", "S", "V", "sq", "grad_sq", "metrics", "ring", "step", "counter"), *runs):
        assert np.array_equal(a, b), name
    assert runs[1][-2][0] == 3 and runs[1][-1][0] == 3
    assert not np.array_equal(runs[1][7][0], np.full(n_metrics, -1.0, np.float32))


def test_clipped_adam_step_with_the_step_end_refuses_a_bad_ring(device):
    from ttrl_amd.engine.tensor import DeviceArray

    lib = _lib.lib()
    x = DeviceArray(device, (8,))
    i = DeviceArray(device, (1,))
    hyper = (C.c_float(1e-3), C.c_float(0.9), C.c_float(0.999), C.c_float(1e-8), C.c_float(0.0))
    base = (device.ctx, x.vp, x.vp, x.vp, x.vp, C.c_long(8), i.vp, *hyper, None, 0, C.c_float(1.0), None, None)
    assert lib.ttrl_adam_step_clipped_end(*base, None, x.vp, 2, x.vp, 1) == _lib.TTRL_EINVAL
    assert lib.ttrl_adam_step_clipped_end(*base, i.vp, None, 2, x.vp, 1) == _lib.TTRL_EINVAL
    assert lib.ttrl_adam_step_clipped_end(*base, i.vp, x.vp, -1, x.vp, 1) == _lib.TTRL_EINVAL
