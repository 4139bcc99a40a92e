"""Float64 forward/backward of the networks on the path.

Nature-CNN Q network   ttrl/nets/encoders.py:86-137, ttrl/nets/towers.py:40,
                       ttrl/nets/heads.py:33-41; forward as the numpy deploy path
                       computes it (ttrl/deploy/conv.py:31-50,
                       ttrl/deploy/artifact.py:188-203): NCHW frames -> NHWC,
                       conv+ReLU x3, flatten in HWC order, Linear+ReLU, Linear.
MLP towers             ttrl/nets/encoders.py:147-172 (Linear+ReLU per hidden
                       width), Linear y = x @ W + b with W (in, out)
                       (ttrl/engine/layers.py:22-61).

ReLU gates: where a float64 pre-activation lies within `band` times the
tensor's RMS of zero, fp32 cannot decide its sign; a caller may pass the
device's gate pattern for such a site and the oracle adopts it there only
(the reference's DeviceGates, tests/_fakes/torch_twin.py:41-168).  Adoptions
and disagreements outside the band are counted in `stats`.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from oracle import conv, fa, float_type

KINK_BAND = 1e-4


@dataclass
class GateStats:
    adopted: dict = field(default_factory=dict)
    decided_mismatch: dict = field(default_factory=dict)


def gate(name: str, z: np.ndarray, gates: dict | None, stats: GateStats | None, band: float = KINK_BAND):
    m = z > 0.0
    if gates is None or name not in gates:
        return m
    dev = np.asarray(gates[name]).reshape(z.shape).astype(bool)
    scale = max(float(np.sqrt(np.mean(z * z))), 1e-30)
    near = np.abs(z) <= band * scale
    if stats is not None:
        stats.adopted[name] = int(np.sum(near & (dev != m)))
        stats.decided_mismatch[name] = int(np.sum(~near & (dev != m)))
    return np.where(near, dev, m)


@dataclass
class QNet:
    convs: list  # [(W oihw, b (O,), stride, padding)]
    fcs: list  # [(W (in, out), b (out,))]; every fc but the last has a ReLU
    scale: float = 1.0 / 255.0

    def copy(self) -> "QNet":
        return QNet([(w.copy(), b.copy(), s, p) for w, b, s, p in self.convs],
                    [(w.copy(), b.copy()) for w, b in self.fcs], self.scale)

    def flat(self) -> list:
        out = []
        for w, b, _, _ in self.convs:
            out += [w, b]
        for w, b in self.fcs:
            out += [w, b]
        return out

    def with_flat(self, flat: list) -> "QNet":
        it = iter(flat)
        convs = [(next(it), next(it), s, p) for _, _, s, p in self.convs]
        fcs = [(next(it), next(it)) for _ in self.fcs]
        return QNet(convs, fcs, self.scale)


def qnet_forward(net: QNet, frames: np.ndarray, *, gates=None, stats=None, prefix: str = ""):
    """-> (q (B, A), acts); acts holds (input, pre-activation, gate) per layer."""
    x = fa(frames)
    h = x.transpose(0, 2, 3, 1) * net.scale
    acts = []
    for i, (w, b, s, p) in enumerate(net.convs):
        z = conv.forward(h, w, b, s, p)
        m = gate(f"{prefix}conv{i}", z, gates, stats)
        acts.append((h, z, m))
        h = z * m
    h = h.reshape(h.shape[0], -1)
    last = len(net.fcs) - 1
    for j, (w, b) in enumerate(net.fcs):
        z = h @ w + b.reshape(1, -1)
        if j < last:
            m = gate(f"{prefix}fc{j}", z, gates, stats)
            acts.append((h, z, m))
            h = z * m
        else:
            acts.append((h, z, None))
            h = z
    return h, acts


def qnet_backward(net: QNet, acts, dq: np.ndarray) -> list:
    """Gradients in `QNet.flat()` order for upstream dL/dq."""
    g = fa(dq)
    nconv = len(net.convs)
    fc_grads = []
    for j in range(len(net.fcs) - 1, -1, -1):
        h_in, _, m = acts[nconv + j]
        if m is not None:
            g = g * m
        w = net.fcs[j][0]
        fc_grads.append((h_in.T @ g, g.sum(axis=0)))
        g = g @ w.T
    fc_grads.reverse()
    conv_grads = []
    if nconv:
        _, z_last, _ = acts[nconv - 1]
        g = g.reshape(z_last.shape)
        for i in range(nconv - 1, -1, -1):
            h_in, _, m = acts[i]
            g = g * m
            w, _, s, p = net.convs[i]
            dx, dw, db = conv.backward(h_in, w, g, s, p, need_dx=i > 0)
            conv_grads.append((dw, db))
            g = dx
        conv_grads.reverse()
    out = []
    for dw, db in conv_grads:
        out += [dw, db]
    for dw, db in fc_grads:
        out += [dw, db]
    return out


def mlp_forward(layers: list, x: np.ndarray, *, relu_last: bool = False, gates=None, stats=None, prefix=""):
    """Linear (+ReLU on all but the last unless relu_last) -> (out, acts)."""
    h = fa(x)
    acts = []
    last = len(layers) - 1
    for j, (w, b) in enumerate(layers):
        z = h @ w + b.reshape(1, -1)
        if j < last or relu_last:
            m = gate(f"{prefix}{j}", z, gates, stats)
            acts.append((h, z, m))
            h = z * m
        else:
            acts.append((h, z, None))
            h = z
    return h, acts


def mlp_backward(layers: list, acts, dout: np.ndarray, *, need_dx: bool = False):
    """-> ([(dW, db) per layer], dx | None)."""
    g = fa(dout)
    grads = []
    for j in range(len(layers) - 1, -1, -1):
        h_in, _, m = acts[j]
        if m is not None:
            g = g * m
        grads.append((h_in.T @ g, g.sum(axis=0)))
        if j > 0 or need_dx:
            g = g @ layers[j][0].T
    grads.reverse()
    return grads, (g if need_dx else None)
