"""The GRU oracle (oracle/gru.py) pinned on the CPU against torch float64:
torch.nn.GRUCell with the transposed stacked weights (which fixes the gate
order and the reset gate's placement to PyTorch's, as the reference's own
parity test does, ttrl/engine/recurrent.py:32-37) unrolled with the done
mask on the entering state, and autograd for every gradient."""

from __future__ import annotations

import numpy as np
import pytest


@pytest.mark.parametrize("T,B,F,H,with_done", [(6, 3, 5, 4, True), (4, 2, 3, 7, False)])
def test_gru_oracle_matches_torch(T, B, F, H, with_done):
    import torch

    from oracle.gru import gru_backward, gru_forward

    rng = np.random.default_rng(T * 10 + H)
    W_ih = rng.uniform(-0.5, 0.5, (F, 3 * H))
    W_hh = rng.uniform(-0.5, 0.5, (H, 3 * H))
    b_ih = rng.uniform(-0.5, 0.5, 3 * H)
    b_hh = rng.uniform(-0.5, 0.5, 3 * H)
    x = rng.standard_normal((T, B, F))
    h0 = rng.standard_normal((B, H))
    done = (rng.random((T, B)) < 0.3).astype(np.float64) if with_done else None
    G = rng.standard_normal((T, B, H))
    outs, cache = gru_forward(W_ih, W_hh, b_ih, b_hh, x, h0, done)
    grads = gru_backward(cache, G)

    cell = torch.nn.GRUCell(F, H).double()
    with torch.no_grad():
        cell.weight_ih.copy_(torch.tensor(W_ih.T))
        cell.weight_hh.copy_(torch.tensor(W_hh.T))
        cell.bias_ih.copy_(torch.tensor(b_ih))
        cell.bias_hh.copy_(torch.tensor(b_hh))
    xt = torch.tensor(x, requires_grad=True)
    ht = torch.tensor(h0, requires_grad=True)
    h, outs_t = ht, []
    for t in range(T):
        if done is not None:
            h = h * (1.0 - torch.tensor(done[t]).reshape(B, 1))
        h = cell(xt[t], h)
        outs_t.append(h)
    out_t = torch.stack(outs_t)
    (out_t * torch.tensor(G)).sum().backward()
    assert np.allclose(outs, out_t.detach().numpy(), rtol=1e-12, atol=1e-12)
    want = [xt.grad.numpy(), ht.grad.numpy(), cell.weight_ih.grad.numpy().T, cell.weight_hh.grad.numpy().T,
            cell.bias_ih.grad.numpy(), cell.bias_hh.grad.numpy()]
    for g, w in zip(grads, want):
        assert np.allclose(g, w, rtol=1e-10, atol=1e-12)
