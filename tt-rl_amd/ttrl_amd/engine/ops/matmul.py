"""matmul on the FP32 MFMA core with the transposed-product backward
(ttrl/engine/ops/matmul.py:55-86).  Full fp32 products and fp32 accumulation:
unlike the reference's HiFi4 path there is no bf16-granularity pass."""

from __future__ import annotations

from ttrl_amd.engine.autograd import Tensor, _detached, _needs
from ttrl_amd.engine.ops import _kernels as K


def purge_matmul_caches(device) -> None:
    """No per-device matmul state is cached; kept for interface parity."""


def matmul(a: Tensor, b: Tensor) -> Tensor:
    """(M, K) @ (K, N) -> (M, N)."""
    if len(a.shape) < 2 or len(b.shape) < 2:
        raise ValueError(
            f"matmul expects rank>=2 operands, got {a.shape} @ {b.shape}; "
            "reshape vectors to an explicit (1, K) / (K, 1) matrix first."
        )
    if len(a.shape) != 2 or len(b.shape) != 2:
        raise ValueError(f"matmul: batched operands are not supported, got {a.shape} @ {b.shape}")
    y = K.matmul_raw(a.data, b.data)
    if not _needs(a, b):
        return _detached(y)
    out = Tensor(y, True, (a, b), "matmul")
    a_data, b_data = a.data, b.data

    def _backward(grad):
        if a.requires_grad:
            a._accumulate(K.matmul_raw(grad, b_data, tb=True))
        if b.requires_grad:
            b._accumulate(K.matmul_raw(a_data, grad, ta=True))

    out._backward = _backward
    return out
