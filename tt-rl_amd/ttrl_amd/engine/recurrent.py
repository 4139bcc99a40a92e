"""`GRUCell` and `GRU` (ttrl/engine/recurrent.py:39-168): one gated recurrent
step, and a fixed-length unroll with episode resets.

Same parameters, layouts and init as the reference: weight_ih (features,
3 * hidden), weight_hh (hidden, 3 * hidden), bias_ih and bias_hh (1,
3 * hidden), gates stacked reset | update | candidate (PyTorch's order),
uniform on +-1/sqrt(hidden) drawn weight_ih, weight_hh, bias_ih, bias_hh.

The unroll is one tape node built for the MI355X: the input projection of
every timestep is one GEMM before the loop; each step is one GEMM (h W_hh +
b_hh) and one fused gate kernel, which also writes the next step's reset
state h * (1 - done); the backward walks the steps in reverse with one fused
gate-gradient kernel and one GEMM (d gh W_hh^T) per step, and the weight and
input gradients of all timesteps come from two GEMM launches at the end
(each W's gradient summed over T in the GEMM's K loop rather than
accumulated T times).
"""

from __future__ import annotations

import ctypes as C
import math

import numpy as np

from ttrl_amd import _lib
from ttrl_amd.engine.autograd import Tensor, _detached, _needs, relu_mask
from ttrl_amd.engine.nn import Module
from ttrl_amd.engine.ops.fused import grad_targets
from ttrl_amd.engine.tensor import DeviceArray

__all__ = ["GATES", "GRU", "GRUCell"]

GATES = ("reset", "update", "candidate")


class GRUCell(Module):
    """One gated recurrent step, (x, h) -> h'."""

    def __init__(self, in_features: int, hidden_size: int, device):
        if in_features <= 0 or hidden_size <= 0:
            raise ValueError(f"GRUCell: in_features and hidden_size must be > 0, got in_features={in_features}, "
                             f"hidden_size={hidden_size}")
        self.in_features = int(in_features)
        self.hidden_size = int(hidden_size)
        gates = len(GATES) * self.hidden_size
        bound = 1.0 / math.sqrt(self.hidden_size)

        def uniform(shape):
            return np.random.uniform(-bound, bound, shape).astype(np.float32)

        self.weight_ih = Tensor.from_numpy(uniform((self.in_features, gates)), device, requires_grad=True)
        self.weight_hh = Tensor.from_numpy(uniform((self.hidden_size, gates)), device, requires_grad=True)
        self.bias_ih = Tensor.from_numpy(uniform((1, gates)), device, requires_grad=True)
        self.bias_hh = Tensor.from_numpy(uniform((1, gates)), device, requires_grad=True)

    def forward(self, x: Tensor, h: Tensor) -> Tensor:
        x_shape, h_shape = tuple(int(d) for d in x.shape), tuple(int(d) for d in h.shape)
        if len(x_shape) != 2 or x_shape[1] != self.in_features:
            raise ValueError(f"GRUCell({self.in_features}, {self.hidden_size}): expected an input of shape "
                             f"(batch, {self.in_features}), got {x_shape}")
        if len(h_shape) != 2 or h_shape[1] != self.hidden_size:
            raise ValueError(f"GRUCell({self.in_features}, {self.hidden_size}): expected a state of shape "
                             f"(batch, {self.hidden_size}), got {h_shape}")
        if x_shape[0] != h_shape[0]:
            raise ValueError(f"GRUCell: input batch {x_shape[0]} and state batch {h_shape[0]} disagree")
        outputs, _ = unroll(self, _reshape_node(x, (1,) + x_shape), h, None)
        return _reshape_node(outputs, h_shape)


class GRU(Module):
    """A GRUCell unrolled over (T, batch, features); `forward(x, h0, done)`
    returns the (T, batch, hidden) outputs and the final state.  `done`
    (T, batch, 1) resets the state entering each timestep."""

    def __init__(self, in_features: int, hidden_size: int, device):
        self.cell = GRUCell(in_features, hidden_size, device)
        self.in_features = self.cell.in_features
        self.hidden_size = self.cell.hidden_size

    def forward(self, x: Tensor, h0: Tensor, done: Tensor | None = None):
        shape = tuple(int(d) for d in x.shape)
        if len(shape) != 3 or shape[2] != self.in_features:
            raise ValueError(f"GRU({self.in_features}, {self.hidden_size}): expected a sequence of shape "
                             f"(timesteps, batch, {self.in_features}), got {shape}. Stack the timesteps on axis 0.")
        steps, batch, _ = shape
        if done is not None and tuple(int(d) for d in done.shape) != (steps, batch, 1):
            raise ValueError(f"GRU: done must be shaped ({steps}, {batch}, 1) to match the sequence it masks, "
                             f"got {tuple(done.shape)}.")
        h_shape = tuple(int(d) for d in h0.shape)
        if h_shape != (batch, self.hidden_size):
            raise ValueError(f"GRU: h0 must be shaped ({batch}, {self.hidden_size}), got {h_shape}")
        return unroll(self.cell, x, h0, done)


def _reshape_node(t: Tensor, shape) -> Tensor:
    data = t.data.reshape(shape)
    if not t.requires_grad:
        return _detached(data)
    out = Tensor(data, True, (t,), "reshape")
    out._backward = lambda grad: t._accumulate(grad.reshape(t.shape))
    return out


def _linear(dev, x: DeviceArray, w: Tensor, b: Tensor, y: DeviceArray, M: int, K: int, N: int) -> None:
    desc = _lib.LinearDesc()
    desc.M, desc.K, desc.N, desc.groups = M, K, N, 1
    desc.x, desc.ldx = x.ptr, K
    desc.W, desc.b = w.data.ptr, b.data.ptr
    desc.y = y.ptr
    dev.call("ttrl_linear_forward", C.byref(desc))


def unroll(cell: GRUCell, x: Tensor, h0: Tensor, done: Tensor | None):
    """-> (outputs (T, B, H), final state (B, H)) as tape tensors."""
    dev = x.device
    T, B, F = (int(d) for d in x.shape)
    H = cell.hidden_size
    G = 3 * H
    X = x.data.reshape((T * B, F))
    GI = DeviceArray(dev, (T, B, G))
    GH = DeviceArray(dev, (T, B, G))
    HIN = DeviceArray(dev, (T, B, H))
    OUT = DeviceArray(dev, (T, B, H))
    dptr = None if done is None else done.data.ptr

    def done_at(t):
        return None if dptr is None else C.c_void_p(dptr + 4 * t * B)

    def at(arr, t, width):
        return arr.view(t * B * width, (B, width))

    W_hh = cell.weight_hh.data
    # One launch per step when the fused kernels' layout holds (H a multiple
    # of 16, float4-aligned operands), else a GEMM and a cell kernel per step.
    fused = H % 16 == 0 and H <= 8192 and all(a.ptr % 16 == 0 for a in (HIN, W_hh))
    _linear(dev, X, cell.weight_ih, cell.bias_ih, GI, T * B, F, G)
    dev.call("ttrl_gru_mask", B, H, h0.data.vp, done_at(0), HIN.vp)
    for t in range(T):
        gi, gh, hin, out = at(GI, t, G), at(GH, t, G), at(HIN, t, H), at(OUT, t, H)
        last = t + 1 == T
        done_next = None if last else done_at(t + 1)
        hin_next = None if last else at(HIN, t + 1, H).vp
        if fused:
            dev.call("ttrl_gru_step_fused", B, H, gi.vp, hin.vp, W_hh.vp, cell.bias_hh.data.vp, gh.vp, out.vp,
                     done_next, hin_next)
        else:
            _linear(dev, hin, cell.weight_hh, cell.bias_hh, gh, B, H, G)
            dev.call("ttrl_gru_step", B, H, gi.vp, gh.vp, hin.vp, out.vp, done_next, hin_next)
    params = (cell.weight_ih, cell.weight_hh, cell.bias_ih, cell.bias_hh)
    final_data = OUT.view((T - 1) * B * H, (B, H))
    if not _needs(x, h0, *params):
        return _detached(OUT), _detached(final_data)
    outputs = Tensor(OUT, True, (x, h0) + params, "gru_unroll")

    def _backward_fused(grad: DeviceArray, DGI: DeviceArray, DGH: DeviceArray, need_h0: bool):
        """The reverse walk with one launch per step: step s's launch forms
        d hin_s and the cell backward of step s - 1; -> d hin_0 or None."""
        DHZ = [DeviceArray(dev, (B, H)), DeviceArray(dev, (B, H))]
        last = T - 1
        dev.call("ttrl_gru_step_backward", B, H, at(GI, last, G).vp, at(GH, last, G).vp, at(HIN, last, H).vp,
                 at(grad, last, H).vp, None, None, at(DGI, last, G).vp, at(DGH, last, G).vp, DHZ[last % 2].vp)
        for s in range(last, 0, -1):
            dev.call("ttrl_gru_step_backward_fused", B, H, at(DGH, s, G).vp, W_hh.vp, DHZ[s % 2].vp, None,
                     at(GI, s - 1, G).vp, at(GH, s - 1, G).vp, at(HIN, s - 1, H).vp, at(grad, s - 1, H).vp,
                     done_at(s), at(DGI, s - 1, G).vp, at(DGH, s - 1, G).vp, DHZ[(s - 1) % 2].vp)
        if not need_h0:
            return None
        dhin0 = DeviceArray(dev, (B, H))
        dev.call("ttrl_gru_step_backward_fused", B, H, at(DGH, 0, G).vp, W_hh.vp, DHZ[0].vp, dhin0.vp,
                 None, None, None, None, None, None, None, None)
        return dhin0

    def _backward(grad: DeviceArray):
        DGI = DeviceArray(dev, (T, B, G))
        DGH = DeviceArray(dev, (T, B, G))
        need_h0 = h0.requires_grad
        if fused:
            dhin0 = _backward_fused(grad, DGI, DGH, need_h0)
        else:
            dhin0 = _backward_steps(grad, DGI, DGH, need_h0)
        if need_h0:
            dh0 = DeviceArray(dev, (B, H))
            dev.call("ttrl_gru_mask", B, H, dhin0.vp, done_at(0), dh0.vp)
            h0._accumulate(dh0)
        _weight_grads(DGI, DGH)

    def _backward_steps(grad: DeviceArray, DGI: DeviceArray, DGH: DeviceArray, need_h0: bool):
        """The reverse walk with a cell-backward kernel and a GEMM per step."""
        DH = [DeviceArray(dev, (B, H)), DeviceArray(dev, (B, H))]
        for t in range(T - 1, -1, -1):
            first = t == T - 1
            cur, nxt = DH[t % 2], DH[(t + 1) % 2]
            dev.call("ttrl_gru_step_backward", B, H, GI.view(t * B * G, (B, G)).vp, GH.view(t * B * G, (B, G)).vp,
                     HIN.view(t * B * H, (B, H)).vp, grad.view(t * B * H, (B, H)).vp, None if first else nxt.vp,
                     None if first else done_at(t + 1), DGI.view(t * B * G, (B, G)).vp,
                     DGH.view(t * B * G, (B, G)).vp, cur.vp)
            if t > 0 or need_h0:
                # d hin_t += d gh_t W_hh^T
                dev.call("ttrl_matmul", B, H, G, DGH.view(t * B * G, (B, G)).vp, C.c_long(G), 0,
                         cell.weight_hh.data.vp, C.c_long(G), 1, cur.vp, C.c_long(H), C.c_float(1.0),
                         C.c_float(1.0))
        return DH[0] if need_h0 else None

    def _weight_grads(DGI: DeviceArray, DGH: DeviceArray):
        (dw_ih, dw_hh, db_ih, db_hh), beta_w = grad_targets(*params)
        (dx,), beta_x = grad_targets(x)
        xmask = relu_mask(x) if dx is not None else None
        for xin, K, dy, dw, db, dxo, bx in ((HIN, H, DGH, dw_hh, db_hh, None, 0.0),
                                             (X, F, DGI, dw_ih, db_ih, dx, beta_x)):
            if dw is None and dxo is None:
                continue
            b = _lib.LinearDesc()
            b.M, b.K, b.N, b.groups = T * B, K, G, 1
            b.x, b.ldx = xin.ptr, K
            b.W = (cell.weight_hh if xin is HIN else cell.weight_ih).data.ptr
            b.dy = dy.ptr
            b.dW = None if dw is None else dw.ptr
            b.db = None if db is None else db.ptr
            b.dx = None if dxo is None else dxo.ptr
            b.lddx = K
            b.dxmask = None if (dxo is None or xmask is None) else xmask.ptr
            b.beta_w, b.beta_x = beta_w, bx
            dev.call("ttrl_linear_backward", C.byref(b))
        if dx is not None:
            x._note_write(beta_x, xmask is not None)

    outputs._backward = _backward
    final = Tensor(final_data, True, (outputs,), "gru_final")

    def _final_backward(grad: DeviceArray):
        full = DeviceArray(dev, (T, B, H))
        full.fill(0.0)
        full.view((T - 1) * B * H, (B, H)).copy_from(grad.reshape((B, H)))
        outputs._accumulate(full)

    final._backward = _final_backward
    return outputs, final
