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
