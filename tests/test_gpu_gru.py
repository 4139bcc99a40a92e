"""The GRU unroll (ttrl/engine/recurrent.py:39-168) on the GPU against the
float64 oracle (oracle/gru.py, itself pinned to torch.nn.GRUCell): outputs,
final state, and the gradients of the input sequence, the initial state and
all four parameters for a random upstream gradient, with and without episode
resets.  Tolerance rel 1e-4 (max abs error over the tensor relative to its
max |value|) after up to 32 timesteps of fp32 recurrence."""

from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _rel(got, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


@pytest.mark.parametrize("T,B,F,H,with_done", [(5, 3, 7, 10, True), (32, 16, 512, 512, True),
                                                (8, 4, 64, 32, False)])
def test_gru_unroll_matches_oracle(device, T, B, F, H, with_done):
    from oracle.gru import gru_backward, gru_forward
    from ttrl_amd.engine.autograd import Tensor
    from ttrl_amd.engine.recurrent import GRU
    from ttrl_amd.engine.tensor import DeviceArray

    np.random.seed(T + H)
    gru = GRU(F, H, device)
    cell = gru.cell
    W_ih, W_hh = cell.weight_ih.numpy(), cell.weight_hh.numpy()
    b_ih, b_hh = cell.bias_ih.numpy().reshape(-1), cell.bias_hh.numpy().reshape(-1)
    rng = np.random.default_rng(T * 100 + B)
    x = rng.standard_normal((T, B, F)).astype(np.float32)
    h0 = rng.standard_normal((B, H)).astype(np.float32)
    done = (rng.random((T, B, 1)) < 0.1).astype(np.float32) if with_done else None
    G = rng.standard_normal((T, B, H)).astype(np.float32)
    xt = Tensor.from_numpy(x, device, requires_grad=True)
    ht = Tensor.from_numpy(h0, device, requires_grad=True)
    dt = None if done is None else Tensor.from_numpy(done, device)
    outs, final = gru(xt, ht, dt)
    ref, cache = gru_forward(W_ih.astype(np.float64), W_hh.astype(np.float64), b_ih, b_hh, x, h0,
                             None if done is None else done.reshape(T, B))
    assert _rel(outs.numpy(), ref) < 1e-4
    assert _rel(final.numpy(), ref[-1]) < 1e-4
    # d/d outputs of sum(outputs * G): the node's backward with G as its seed.
    seed = DeviceArray(device, (T, B, H))
    seed.upload(G)
    outs.grad = seed
    outs._grad_owned = True
    outs._backward(seed)
    want = gru_backward(cache, G)
    got = [xt.grad.numpy(), ht.grad.numpy(), cell.weight_ih.grad.numpy(), cell.weight_hh.grad.numpy(),
           cell.bias_ih.grad.numpy().reshape(-1), cell.bias_hh.grad.numpy().reshape(-1)]
    for name, g, w in zip(("dx", "dh0", "dW_ih", "dW_hh", "db_ih", "db_hh"), got, want):
        assert _rel(g, w) < 1e-4, name


def test_gru_cell_single_step(device):
    from oracle.gru import gru_forward
    from ttrl_amd.engine.autograd import Tensor
    from ttrl_amd.engine.recurrent import GRUCell

    np.random.seed(3)
    cell = GRUCell(6, 5, device)
    rng = np.random.default_rng(4)
    x = rng.standard_normal((4, 6)).astype(np.float32)
    h = rng.standard_normal((4, 5)).astype(np.float32)
    y = cell(Tensor.from_numpy(x, device), Tensor.from_numpy(h, device)).numpy()
    ref, _ = gru_forward(cell.weight_ih.numpy().astype(np.float64), cell.weight_hh.numpy().astype(np.float64),
                         cell.bias_ih.numpy().reshape(-1), cell.bias_hh.numpy().reshape(-1), x[None], h)
    assert y.shape == (4, 5) and _rel(y, ref[0]) < 1e-5
    with pytest.raises(ValueError, match="expected an input of shape"):
        cell(Tensor.from_numpy(x[:, :5], device), Tensor.from_numpy(h, device))


def _arr(device, a):
    from ttrl_amd.engine.tensor import DeviceArray

    d = DeviceArray(device, a.shape)
    d.upload(np.ascontiguousarray(a, np.float32))
    return d


def _sig(x):
    return 1.0 / (1.0 + np.exp(-x))


@pytest.mark.parametrize("B,H", [(16, 512), (20, 48), (3, 16), (33, 32)])
def test_fused_steps_match_the_two_launch_steps(device, B, H):
    """ttrl_gru_step_fused / ttrl_gru_step_backward_fused against the GEMM +
    cell-kernel steps and a float64 restatement of one timestep (the cell of
    ttrl/engine/recurrent.py:86-94 and its backward), ragged batches included.
    The products sum in another order, so the bound is rel 1e-5."""
    import ctypes as C

    from ttrl_amd import _lib
    from ttrl_amd.engine.tensor import DeviceArray

    G = 3 * H
    rng = np.random.default_rng(B * 1000 + H)
    gi = rng.standard_normal((B, G)).astype(np.float32)
    hin = rng.standard_normal((B, H)).astype(np.float32)
    W = (rng.standard_normal((H, G)) / np.sqrt(H)).astype(np.float32)
    b = rng.standard_normal((1, G)).astype(np.float32)
    done = (rng.random(B) < 0.3).astype(np.float32)

    # forward, float64
    gh64 = hin.astype(np.float64) @ W + b[0]
    r = _sig(gi[:, :H] + gh64[:, :H])
    z = _sig(gi[:, H:2 * H] + gh64[:, H:2 * H])
    n = np.tanh(gi[:, 2 * H:] + r * gh64[:, 2 * H:])
    out64 = (1 - z) * n + z * hin

    dgi_, dhin_, dW_, db_, ddone = (_arr(device, x) for x in (gi, hin, W, b, done))
    outs = {}
    for fused in (False, True):
        gh, hout, hnext = DeviceArray(device, (B, G)), DeviceArray(device, (B, H)), DeviceArray(device, (B, H))
        if fused:
            device.call("ttrl_gru_step_fused", B, H, dgi_.vp, dhin_.vp, dW_.vp, db_.vp, gh.vp, hout.vp, ddone.vp,
                        hnext.vp)
        else:
            lin = _lib.LinearDesc()  # gh = hin W_hh + b_hh, the unfused unroll's product
            lin.M, lin.K, lin.N, lin.groups = B, H, G, 1
            lin.x, lin.ldx, lin.W, lin.b, lin.y = dhin_.ptr, H, dW_.ptr, db_.ptr, gh.ptr
            device.call("ttrl_linear_forward", C.byref(lin))
            device.call("ttrl_gru_step", B, H, dgi_.vp, gh.vp, dhin_.vp, hout.vp, ddone.vp, hnext.vp)
        outs[fused] = (gh.numpy(), hout.numpy(), hnext.numpy())
    for k, (g_ref, name) in enumerate(((gh64, "gh"), (out64, "hout"), (out64 * (1 - done)[:, None], "hin_next"))):
        assert _rel(outs[True][k], g_ref) < 1e-5, name
        assert _rel(outs[True][k], outs[False][k]) < 1e-5, name

    # backward through step t (d hin_t) and the cell of step t - 1
    dgh = rng.standard_normal((B, G)).astype(np.float32)
    dhz = rng.standard_normal((B, H)).astype(np.float32)
    dout = rng.standard_normal((B, H)).astype(np.float32)
    ghp = outs[True][0]
    dhin64 = dhz + dgh.astype(np.float64) @ W.T.astype(np.float64)
    dh = dout + (1 - done)[:, None] * dhin64
    r = _sig(gi[:, :H] + ghp[:, :H])
    z = _sig(gi[:, H:2 * H] + ghp[:, H:2 * H])
    hn = ghp[:, 2 * H:].astype(np.float64)
    c = np.tanh(gi[:, 2 * H:] + r * hn)
    dcp = dh * (1 - z) * (1 - c * c)
    drp = dcp * hn * r * (1 - r)
    dzp = dh * (hin - c) * z * (1 - z)
    want = {"dhin": dhin64, "dgi": np.concatenate([drp, dzp, dcp], 1),
            "dgh": np.concatenate([drp, dzp, dcp * r], 1), "dhz": dh * z}

    d_dgh, d_dhz, d_dout, d_ghp = (_arr(device, x) for x in (dgh, dhz, dout, ghp))
    got = {}
    for fused in (False, True):
        dhin = DeviceArray(device, (B, H))
        dgi_o, dgh_o, dhz_o = DeviceArray(device, (B, G)), DeviceArray(device, (B, G)), DeviceArray(device, (B, H))
        if fused:
            device.call("ttrl_gru_step_backward_fused", B, H, d_dgh.vp, dW_.vp, d_dhz.vp, dhin.vp, dgi_.vp, d_ghp.vp,
                        dhin_.vp, d_dout.vp, ddone.vp, dgi_o.vp, dgh_o.vp, dhz_o.vp)
        else:
            dhin.upload(dhz)
            device.call("ttrl_matmul", B, H, G, d_dgh.vp, C.c_long(G), 0, dW_.vp, C.c_long(G), 1, dhin.vp,
                        C.c_long(H), C.c_float(1.0), C.c_float(1.0))
            device.call("ttrl_gru_step_backward", B, H, dgi_.vp, d_ghp.vp, dhin_.vp, d_dout.vp, dhin.vp, ddone.vp,
                        dgi_o.vp, dgh_o.vp, dhz_o.vp)
        got[fused] = {"dhin": dhin.numpy(), "dgi": dgi_o.numpy(), "dgh": dgh_o.numpy(), "dhz": dhz_o.numpy()}
    for name, w in want.items():
        assert _rel(got[True][name], w) < 1e-5, name
        assert _rel(got[True][name], got[False][name]) < 1e-5, name

    # d hin only (the walk's last launch, no cell before it)
    only = DeviceArray(device, (B, H))
    device.call("ttrl_gru_step_backward_fused", B, H, d_dgh.vp, dW_.vp, d_dhz.vp, only.vp, None, None, None, None,
                None, None, None, None)
    assert np.array_equal(only.numpy(), got[True]["dhin"])


def test_fused_steps_refuse_what_they_cannot_run(device):
    from ttrl_amd.engine.tensor import DeviceArray

    x = DeviceArray(device, (4 * 3 * 24,))
    with pytest.raises(ValueError, match="multiple of 16"):
        device.call("ttrl_gru_step_fused", 4, 24, x.vp, x.vp, x.vp, x.vp, x.vp, x.vp, None, None)
    with pytest.raises(ValueError, match="given together"):
        device.call("ttrl_gru_step_backward_fused", 4, 16, x.vp, x.vp, x.vp, x.vp, x.vp, None, None, None, None,
                    None, None, None)
