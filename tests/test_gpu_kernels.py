"""Kernel parity on the GPU: every entry point against a float64 reference
on seeded inputs.  fp32 kernels vs float64 math: tolerances are stated per
check (relative to the reference's scale)."""

from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _dev_arr(device, a, dtype=np.float32):
    from ttrl_amd.engine.tensor import to_device
    return to_device(np.asarray(a), device, dtype)


def _rel(got, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


@pytest.mark.parametrize("M,N,K", [(16, 16, 4), (37, 53, 61), (64, 64, 64), (32, 512, 3136), (256, 256, 256),
                                   (1, 7, 3), (300, 5, 1000)])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_matmul_matches_float64(device, M, N, K, ta, tb):
    from ttrl_amd.engine.ops import _kernels as Kk
    rng = np.random.default_rng(M * 1000 + N * 10 + K + 7 * ta + 3 * tb)
    a = rng.standard_normal((K, M) if ta else (M, K)).astype(np.float32)
    b = rng.standard_normal((N, K) if tb else (K, N)).astype(np.float32)
    ref = (a.T if ta else a).astype(np.float64) @ (b.T if tb else b).astype(np.float64)
    got = Kk.matmul_raw(_dev_arr(device, a), _dev_arr(device, b), ta=bool(ta), tb=bool(tb)).numpy()
    # fp32 products, fp32 accumulation over K terms: error ~ sqrt(K) * 2^-24 * |terms|
    assert _rel(got, ref) < 2e-5 * max(1.0, np.sqrt(K) / 8)


def test_linear_forward_backward(device):
    from ttrl_amd import _lib
    from ttrl_amd.engine.tensor import DeviceArray
    rng = np.random.default_rng(1)
    M, K, N = 32, 3136, 512
    x = rng.standard_normal((M, K)).astype(np.float32)
    W = (rng.standard_normal((K, N)) / np.sqrt(K)).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32)
    dy = rng.standard_normal((M, N)).astype(np.float32)
    dx_, dW_, db_, x_, y_ = (DeviceArray(device, s) for s in ((M, K), (K, N), (N,), (M, K), (M, N)))
    xd, Wd, bd, dyd = (_dev_arr(device, v) for v in (x, W, b, dy))
    d = _lib.LinearDesc()
    d.M, d.K, d.N, d.groups = M, K, N, 1
    d.x, d.ldx, d.W, d.b, d.y, d.relu = xd.ptr, K, Wd.ptr, bd.ptr, y_.ptr, 1
    device.call("ttrl_linear_forward", C.byref(d))
    z = x.astype(np.float64) @ W + b
    y_ref = np.maximum(z, 0)
    assert _rel(y_.numpy(), y_ref) < 1e-5
    e = _lib.LinearDesc()
    e.M, e.K, e.N, e.groups = M, K, N, 1
    e.x, e.ldx, e.W, e.dy, e.ymask = xd.ptr, K, Wd.ptr, dyd.ptr, y_.ptr
    e.dW, e.db, e.dx, e.lddx = dW_.ptr, db_.ptr, dx_.ptr, K
    device.call("ttrl_linear_backward", C.byref(e))
    mask = y_.numpy() > 0
    dz = dy.astype(np.float64) * mask
    assert _rel(dW_.numpy(), x.T.astype(np.float64) @ dz) < 1e-5
    assert _rel(db_.numpy(), dz.sum(0)) < 1e-5
    assert _rel(dx_.numpy(), dz @ W.T.astype(np.float64)) < 1e-5
    # The gate of the layer below applied as dx is written (dxmask), with the
    # already-gated dZ passed in and no ymask: same dW, dx * [x > 0].
    dzd = _dev_arr(device, dz.astype(np.float32))
    f = _lib.LinearDesc()
    f.M, f.K, f.N, f.groups = M, K, N, 1
    f.x, f.ldx, f.W, f.dy, f.dxmask = xd.ptr, K, Wd.ptr, dzd.ptr, xd.ptr
    dx2 = DeviceArray(device, (M, K))
    f.dx, f.lddx = dx2.ptr, K
    device.call("ttrl_linear_backward", C.byref(f))
    assert _rel(dx2.numpy(), (dz @ W.T.astype(np.float64)) * (x > 0)) < 1e-5


@pytest.mark.parametrize("case", [
    dict(B=2, C=4, H=84, W=84, O=32, k=8, s=4, p=0, u8=True),
    dict(B=3, C=32, H=20, W=20, O=64, k=4, s=2, p=0, u8=False),
    dict(B=3, C=64, H=9, W=9, O=64, k=3, s=1, p=0, u8=False),
    dict(B=2, C=8, H=8, W=8, O=8, k=3, s=1, p=1, u8=False),
    dict(B=2, C=6, H=11, W=11, O=5, k=3, s=2, p=1, u8=False),
])
def test_conv_forward_and_gradients(device, case):
    from oracle import conv as oconv
    from ttrl_amd import _lib
    from ttrl_amd.engine.conv import oihw_to_master, master_to_oihw
    from ttrl_amd.engine.tensor import DeviceArray
    rng = np.random.default_rng(sum(case.values()))
    B, Cc, H, W, O, k, s, p = (case[n] for n in ("B", "C", "H", "W", "O", "k", "s", "p"))
    u8 = case["u8"]
    OH = (H + 2 * p - k) // s + 1
    OW = (W + 2 * p - k) // s + 1
    w = (rng.standard_normal((O, Cc, k, k)) / np.sqrt(Cc * k * k)).astype(np.float32)
    bias = rng.standard_normal(O).astype(np.float32) * 0.1
    scale = 1.0 / 255.0 if u8 else 1.0
    if u8:
        frames = rng.integers(0, 256, (B, Cc, H, W), dtype=np.uint8)
        x_nhwc = frames.transpose(0, 2, 3, 1).astype(np.float64) * scale
        xd = _dev_arr(device, frames, np.uint8)
        layout = "nchw_u8"
    else:
        x_nhwc = rng.standard_normal((B, H, W, Cc)).astype(np.float32)
        xd = _dev_arr(device, x_nhwc)
        x_nhwc = x_nhwc.astype(np.float64)
        layout = "nhwc"
    wt = oihw_to_master(w, layout)
    assert np.array_equal(master_to_oihw(wt, w.shape, layout), w)
    wd, bd = _dev_arr(device, wt), _dev_arr(device, bias)
    g = _lib.ConvGeom(B, Cc, H, W, O, k, s, p, _lib.LAYOUT_NCHW_U8 if u8 else _lib.LAYOUT_NHWC_F32)
    y = DeviceArray(device, (B, OH, OW, O))
    device.call("ttrl_conv2d_forward", C.byref(g), xd.vp, wd.vp, bd.vp, y.vp, C.c_float(scale), 1)
    z = oconv.forward(x_nhwc, w, bias, s, p)
    assert _rel(y.numpy(), np.maximum(z, 0)) < 2e-5
    dy = rng.standard_normal((B, OH, OW, O)).astype(np.float32)
    dyd = _dev_arr(device, dy)
    dw_ = DeviceArray(device, wt.shape)
    db_ = DeviceArray(device, (O,))
    device.call("ttrl_conv2d_backward_weight", C.byref(g), xd.vp, C.c_float(scale), dyd.vp, y.vp, dw_.vp,
                db_.vp, C.c_float(0.0))
    mask = y.numpy() > 0
    dz = dy.astype(np.float64) * mask
    dx_ref, dw_ref, db_ref = oconv.backward(x_nhwc, w, dz, s, p)
    assert _rel(master_to_oihw(dw_.numpy(), w.shape, layout), dw_ref) < 2e-5
    assert _rel(db_.numpy(), db_ref) < 2e-5
    if not u8:
        dx_ = DeviceArray(device, (B, H, W, Cc))
        device.call("ttrl_conv2d_backward_input", C.byref(g), dyd.vp, y.vp, wd.vp, dx_.vp, None, C.c_float(1.0),
                    C.c_float(0.0))
        assert _rel(dx_.numpy(), dx_ref) < 2e-5
        # Pre-gated dZ, no ymask, and the input's own ReLU gate fused into the write.
        dzd = _dev_arr(device, dz.astype(np.float32))
        dx2 = DeviceArray(device, (B, H, W, Cc))
        device.call("ttrl_conv2d_backward_input", C.byref(g), dzd.vp, None, wd.vp, dx2.vp, xd.vp, C.c_float(1.0),
                    C.c_float(0.0))
        assert _rel(dx2.numpy(), dx_ref * (x_nhwc > 0)) < 2e-5
        # Both gradients in one call (a paired launch), with the output's and
        # the input's ReLU gates and beta accumulation into preset buffers.
        dw3, db3, dx3 = DeviceArray(device, wt.shape), DeviceArray(device, (O,)), DeviceArray(device, (B, H, W, Cc))
        for t in (dw3, db3, dx3):
            t.fill(0.5)
        device.call("ttrl_conv2d_backward", C.byref(g), xd.vp, C.c_float(scale), dyd.vp, y.vp, wd.vp, dw3.vp, db3.vp,
                    C.c_float(1.0), dx3.vp, xd.vp, C.c_float(2.0))
        assert _rel(master_to_oihw(dw3.numpy(), w.shape, layout) - 0.5, dw_ref) < 2e-5
        assert _rel(db3.numpy() - 0.5, db_ref) < 2e-5
        assert _rel(dx3.numpy() - 1.0, dx_ref * (x_nhwc > 0)) < 2e-5


@pytest.mark.parametrize("n", [10007, 2_200_003])
def test_adam_step_matches_fused_oracle_over_steps(device, n):
    """A ragged tail (n % 4), a partial last workgroup, and (2.2M) more
    than one pass of the grid per thread."""
    from oracle import adam as oadam
    from ttrl_amd.engine.tensor import DeviceArray
    rng = np.random.default_rng(3)
    p = rng.uniform(-1, 1, n).astype(np.float32)
    pd = _dev_arr(device, p)
    S, V = DeviceArray(device, (n,)), DeviceArray(device, (n,))
    S.fill(0.0)
    V.fill(0.0)
    t = DeviceArray(device, (1,), np.int32)
    t.fill(0)
    gsq = DeviceArray(device, (1,))
    pr, Sr, Vr = p.astype(np.float64), np.zeros(n), np.zeros(n)
    for step in range(1, 6):
        g = rng.uniform(-0.1, 0.1, n).astype(np.float32)
        gd = _dev_arr(device, g)
        device.call("ttrl_adam_step", pd.vp, gd.vp, S.vp, V.vp, C.c_long(n), t.vp, C.c_float(1e-3),
                    C.c_float(0.9), C.c_float(0.999), C.c_float(1e-8), C.c_float(0.0), gsq.vp, 0)
        pr, Sr, Vr = oadam.fused_step(pr, g, Sr, Vr, step, 1e-3)
        assert abs(float(gsq.numpy()[0]) - float(np.sum(g.astype(np.float64) ** 2))) < 1e-4 * np.sum(g * g)
    assert int(t.numpy()[0]) == 5
    assert np.max(np.abs(pd.numpy() - pr)) < 1e-6


def test_dqn_loss_head_matches_oracle(device):
    from oracle.dqn import huber
    from ttrl_amd.engine.tensor import DeviceArray
    rng = np.random.default_rng(5)
    B, A = 32, 6
    q, qs, qv = (rng.standard_normal((B, A)).astype(np.float32) for _ in range(3))
    actions = rng.integers(0, A, B)
    onehot = np.eye(A, dtype=np.float32)[actions]
    r = rng.choice([-1.0, 0.0, 1.0], B, p=[0.05, 0.9, 0.05]).astype(np.float32)
    d = (rng.random(B) < 0.1).astype(np.float32)
    disc = np.full(B, 0.99 ** 3, np.float32)
    w = rng.uniform(0.4, 1.0, B).astype(np.float32)
    outs = {k: DeviceArray(device, s) for k, s in
            (("loss", (1,)), ("mq", (1,)), ("td", (B,)), ("dq", (B, A)), ("na", (B,)), ("y", (B,)))}
    ins = [_dev_arr(device, v) for v in (q, qs, qv, onehot, r, d, disc, w)]
    device.call("ttrl_dqn_loss", B, A, *[v.vp for v in ins], C.c_float(1.0), outs["loss"].vp, outs["mq"].vp,
                outs["td"].vp, outs["dq"].vp, outs["na"].vp, outs["y"].vp)
    a_star = np.argmax(qs, 1)
    y = r + disc * (1 - d) * qv[np.arange(B), a_star].astype(np.float64)
    pred = q[np.arange(B), actions].astype(np.float64)
    e = pred - y
    assert np.array_equal(outs["na"].numpy().astype(int), a_star)
    assert _rel(outs["y"].numpy(), y) < 1e-6
    assert abs(outs["loss"].numpy()[0] - np.mean(w * huber(e, 1.0))) < 1e-6 * max(1, np.mean(w * huber(e, 1.0)))
    assert abs(outs["mq"].numpy()[0] - pred.mean()) < 1e-6
    dq = np.zeros((B, A))
    dq[np.arange(B), actions] = w / B * np.clip(e, -1, 1)
    assert np.max(np.abs(outs["dq"].numpy() - dq)) < 1e-7
    assert _rel(outs["td"].numpy(), np.abs(e)) < 1e-6


@pytest.mark.parametrize("groups,B,K,A", [(3, 32, 512, 6), (2, 32, 512, 6), (3, 7, 100, 18), (3, 130, 64, 4),
                                           (3, 32, 512, 12), (3, 64, 700, 5), (2, 200, 256, 32)])
def test_dqn_head_fused_matches_linear_then_loss(device, groups, B, K, A):
    """ttrl_dqn_head (last linear layer x groups + DQN loss, one launch)
    against float64: q per group, then the loss head on those q (group 1
    selects, the last group values).  Tolerance: q rel 2e-6 (fp32 dot of
    K terms), loss / dq / targets through the oracle rel 1e-5; argmax
    adopted from the device where the top-two gap is under 1e-5."""
    from oracle.dqn import huber
    from ttrl_amd import _lib
    from ttrl_amd.engine.tensor import DeviceArray
    rng = np.random.default_rng(groups * 1000 + B + K + A)
    hs = [np.maximum(rng.standard_normal((B, K)), 0).astype(np.float32) for _ in range(groups)]
    Ws = [(rng.standard_normal((K, A)) / np.sqrt(K)).astype(np.float32) for _ in range(groups)]
    bs = [(0.1 * rng.standard_normal(A)).astype(np.float32) for _ in range(groups)]
    actions = rng.integers(0, A, B)
    onehot = np.eye(A, dtype=np.float32)[actions]
    r = rng.choice([-1.0, 0.0, 1.0], B, p=[0.1, 0.8, 0.1]).astype(np.float32)
    d = (rng.random(B) < 0.2).astype(np.float32)
    disc = np.full(B, 0.99 ** 3, np.float32)
    w = rng.uniform(0.4, 1.0, B).astype(np.float32)
    hd = [_dev_arr(device, h) for h in hs]
    Wd = [_dev_arr(device, W) for W in Ws]
    bd = [_dev_arr(device, b) for b in bs]
    qd = [DeviceArray(device, (B, A)) for _ in range(groups)]
    outs = {k: DeviceArray(device, s) for k, s in
            (("loss", (1,)), ("mq", (1,)), ("td", (B,)), ("dq", (B, A)), ("na", (B,)), ("y", (B,)))}
    ins = [_dev_arr(device, v) for v in (onehot, r, d, disc, w)]
    # Twice: above 64 samples the batch means are finished by the last
    # workgroup through a device counter that each launch must leave at zero
    # for the next.
    for rep in range(2):
        for o in outs.values():
            o.fill(-7.0)
        device.call("ttrl_dqn_head", B, K, A, groups, _lib.ptrs(x.ptr for x in hd), _lib.ptrs(x.ptr for x in Wd),
                    _lib.ptrs(x.ptr for x in bd), _lib.ptrs(x.ptr for x in qd), *[v.vp for v in ins], C.c_float(1.0),
                    outs["loss"].vp, outs["mq"].vp, outs["td"].vp, outs["dq"].vp, outs["na"].vp, outs["y"].vp)
    q64 = [h.astype(np.float64) @ W + b for h, W, b in zip(hs, Ws, bs)]
    for g in range(groups):
        assert _rel(qd[g].numpy(), q64[g]) < 2e-6
    sel, val = q64[1], q64[groups - 1]
    a_star = np.argmax(sel, 1)
    top2 = np.sort(sel, 1)[:, -2:]
    close = (top2[:, 1] - top2[:, 0]) < 1e-5
    a_dev = outs["na"].numpy().astype(int)
    assert np.array_equal(a_dev[~close], a_star[~close])
    a_star = np.where(close, a_dev, a_star)
    y = r + disc * (1 - d) * val[np.arange(B), a_star]
    pred = q64[0][np.arange(B), actions]
    e = pred - y
    ref_loss = np.mean(w * huber(e, 1.0))
    assert abs(outs["loss"].numpy()[0] - ref_loss) < 1e-5 * max(1.0, abs(ref_loss))
    assert abs(outs["mq"].numpy()[0] - pred.mean()) < 1e-5 * max(1.0, abs(pred.mean()))
    assert _rel(outs["y"].numpy(), y) < 1e-5
    dq = np.zeros((B, A))
    dq[np.arange(B), actions] = w / B * np.clip(e, -1, 1)
    assert np.max(np.abs(outs["dq"].numpy() - dq)) < 1e-5 * max(1e-3, np.abs(dq).max())
