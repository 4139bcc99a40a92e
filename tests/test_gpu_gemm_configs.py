"""Every tile shape of the GEMM core (forced through TTRL_GEMM_FORCE, with and
without split-K) on ragged linear and convolution problems of each loader
kind, against float64, alone and as paired launches (a layer's dW and dX in
one kernel: linear backward and ttrl_conv2d_backward).  A shape a call site does not instantiate falls back
to its normal plan, which is checked the same way.  Tolerance: rel 2e-5 of
each output's scale (fp32 accumulation over at most a few thousand terms)."""

from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

N_CFG = 15
CASES = [(c, s) for c in range(N_CFG) for s in (0, 3)]


def _rel(got, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


def _dev(device, a, dtype=np.float32):
    from ttrl_amd.engine.tensor import to_device
    return to_device(np.ascontiguousarray(a), device, dtype)


@pytest.mark.parametrize("cfg,splits", CASES)
def test_linear_forward_backward_each_tile(device, monkeypatch, cfg, splits):
    from ttrl_amd import _lib
    from ttrl_amd.engine.tensor import DeviceArray
    monkeypatch.setenv("TTRL_GEMM_FORCE", f"{cfg}:{splits}")
    rng = np.random.default_rng(cfg * 10 + splits)
    M, K, N = 37, 300, 70
    x = rng.standard_normal((M, K)).astype(np.float32)
    W = (rng.standard_normal((K, N)) / np.sqrt(K)).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32)
    dz = rng.standard_normal((M, N)).astype(np.float32)
    xd, Wd, bd, dzd = (_dev(device, v) for v in (x, W, b, dz))
    y = DeviceArray(device, (M, N))
    d = _lib.LinearDesc()
    d.M, d.K, d.N, d.groups = M, K, N, 1
    d.x, d.ldx, d.W, d.b, d.y, d.relu = xd.ptr, K, Wd.ptr, bd.ptr, y.ptr, 1
    device.call("ttrl_linear_forward", C.byref(d))
    assert _rel(y.numpy(), np.maximum(x.astype(np.float64) @ W + b, 0)) < 2e-5
    dW, db, dx = DeviceArray(device, (K, N)), DeviceArray(device, (N,)), DeviceArray(device, (M, K))
    e = _lib.LinearDesc()
    e.M, e.K, e.N, e.groups = M, K, N, 1
    e.x, e.ldx, e.W, e.dy = xd.ptr, K, Wd.ptr, dzd.ptr
    e.dW, e.db, e.dx, e.lddx = dW.ptr, db.ptr, dx.ptr, K
    device.call("ttrl_linear_backward", C.byref(e))
    dz64 = dz.astype(np.float64)
    assert _rel(dW.numpy(), x.T.astype(np.float64) @ dz64) < 2e-5
    assert _rel(db.numpy(), dz64.sum(0)) < 2e-5
    assert _rel(dx.numpy(), dz64 @ W.T.astype(np.float64)) < 2e-5


@pytest.mark.parametrize("cfg,splits", CASES)
@pytest.mark.parametrize("u8", [True, False])
def test_conv_each_tile(device, monkeypatch, cfg, splits, u8):
    from oracle import conv as oconv
    from ttrl_amd import _lib
    from ttrl_amd.engine.conv import oihw_to_master, master_to_oihw
    from ttrl_amd.engine.tensor import DeviceArray
    monkeypatch.setenv("TTRL_GEMM_FORCE", f"{cfg}:{splits}")
    rng = np.random.default_rng(100 + cfg * 10 + splits + u8)
    if u8:
        B, Cc, H, W, O, k, s, p = 3, 4, 84, 84, 32, 8, 4, 0
    else:
        B, Cc, H, W, O, k, s, p = 3, 32, 20, 20, 64, 4, 2, 0
    OH = (H + 2 * p - k) // s + 1
    w = (rng.standard_normal((O, Cc, k, k)) / np.sqrt(Cc * k * k)).astype(np.float32)
    bias = (0.1 * rng.standard_normal(O)).astype(np.float32)
    if u8:
        frames = rng.integers(0, 256, (B, Cc, H, W), dtype=np.uint8)
        x64 = frames.transpose(0, 2, 3, 1).astype(np.float64) / 255.0
        xd, layout, scale = _dev(device, frames, np.uint8), "nchw_u8", 1.0 / 255.0
    else:
        xf = rng.standard_normal((B, H, W, Cc)).astype(np.float32)
        x64, xd, layout, scale = xf.astype(np.float64), _dev(device, xf), "nhwc", 1.0
    wt = oihw_to_master(w, layout)
    wd, bd = _dev(device, wt), _dev(device, bias)
    g = _lib.ConvGeom(B, Cc, H, W, O, k, s, p, _lib.LAYOUT_NCHW_U8 if u8 else _lib.LAYOUT_NHWC_F32)
    y = DeviceArray(device, (B, OH, OH, O))
    device.call("ttrl_conv2d_forward", C.byref(g), xd.vp, wd.vp, bd.vp, y.vp, C.c_float(scale), 0)
    assert _rel(y.numpy(), oconv.forward(x64, w, bias, s, p)) < 2e-5
    dz = rng.standard_normal((B, OH, OH, O)).astype(np.float32)
    dzd = _dev(device, dz)
    dw, db = DeviceArray(device, wt.shape), DeviceArray(device, (O,))
    device.call("ttrl_conv2d_backward_weight", C.byref(g), xd.vp, C.c_float(scale), dzd.vp, None, dw.vp, db.vp,
                C.c_float(0.0))
    dx_ref, dw_ref, db_ref = oconv.backward(x64, w, dz.astype(np.float64), s, p)
    assert _rel(master_to_oihw(dw.numpy(), w.shape, layout), dw_ref) < 2e-5
    assert _rel(db.numpy(), db_ref) < 2e-5
    if not u8:
        dx = DeviceArray(device, (B, H, W, Cc))
        device.call("ttrl_conv2d_backward_input", C.byref(g), dzd.vp, None, wd.vp, dx.vp, None, C.c_float(1.0),
                    C.c_float(0.0))
        assert _rel(dx.numpy(), dx_ref) < 2e-5
        # both gradients in one paired launch
        dw2, db2, dx2 = DeviceArray(device, wt.shape), DeviceArray(device, (O,)), DeviceArray(device, (B, H, W, Cc))
        device.call("ttrl_conv2d_backward", C.byref(g), xd.vp, C.c_float(scale), dzd.vp, None, wd.vp, dw2.vp, db2.vp,
                    C.c_float(0.0), dx2.vp, None, C.c_float(0.0))
        assert _rel(master_to_oihw(dw2.numpy(), w.shape, layout), dw_ref) < 2e-5
        assert _rel(db2.numpy(), db_ref) < 2e-5
        assert _rel(dx2.numpy(), dx_ref) < 2e-5


@pytest.mark.parametrize("B", [32, 256])
def test_conv_backward_choice_gives_the_separate_gradients(device, B):
    """ttrl_conv2d_backward runs the pair or two launches, whichever it
    measured faster for the geometry; either way it gives the gradients of
    ttrl_conv2d_backward_weight and ttrl_conv2d_backward_input (rel 1e-5: the
    plans may sum in another order), with beta accumulation and the ReLU
    gates, and files its choice with the context's plans."""
    from ttrl_amd import _lib
    from ttrl_amd.engine.tensor import DeviceArray

    Cin, H, O, k, s = 32, 20, 64, 4, 2
    OH = (H - k) // s + 1
    g = _lib.ConvGeom(B, Cin, H, H, O, k, s, 0, _lib.LAYOUT_NHWC_F32)
    rng = np.random.default_rng(B)
    x = rng.standard_normal((B, H, H, Cin)).astype(np.float32)
    dy = rng.standard_normal((B, OH, OH, O)).astype(np.float32)
    ymask = rng.standard_normal((B, OH, OH, O)).astype(np.float32)
    wt = (0.1 * rng.standard_normal((k * k * Cin, O))).astype(np.float32)
    xd, dyd, md, wd = (_dev(device, a) for a in (x, dy, ymask, wt))
    dw, db, dx = DeviceArray(device, wt.shape), DeviceArray(device, (O,)), DeviceArray(device, x.shape)
    device.call("ttrl_conv2d_backward_weight", C.byref(g), xd.vp, C.c_float(1.0), dyd.vp, md.vp, dw.vp, db.vp,
                C.c_float(0.0))
    device.call("ttrl_conv2d_backward_input", C.byref(g), dyd.vp, md.vp, wd.vp, dx.vp, xd.vp, C.c_float(1.0),
                C.c_float(0.0))
    dw2, db2, dx2 = DeviceArray(device, wt.shape), DeviceArray(device, (O,)), DeviceArray(device, x.shape)
    for t in (dw2, db2, dx2):
        t.fill(0.5)
    for rep in range(2):  # the first call chooses, the second runs the kept choice
        device.call("ttrl_conv2d_backward", C.byref(g), xd.vp, C.c_float(1.0), dyd.vp, md.vp, wd.vp, dw2.vp, db2.vp,
                    C.c_float(1.0), dx2.vp, xd.vp, C.c_float(1.0))
    assert _rel(dw2.numpy() - 0.5, 2 * dw.numpy()) < 1e-5
    assert _rel(db2.numpy() - 0.5, 2 * db.numpy()) < 1e-5
    assert _rel(dx2.numpy() - 0.5, 2 * dx.numpy()) < 1e-5
    assert f"ttrl_conv2d_backward:pair|" in device.export_plans()
