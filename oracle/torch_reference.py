"""The reference's torch CPU paths timed as CPU columns (config 4, the conv row) — TEST INFRASTRUCTURE.

A restatement of tsfast's constant-matrix ``linear_recurrence`` op as the reference computes it
on the CPU (tsfast/models/architectures/dynonet/core.py:23-88): a log-doubling scan (each level
adds the state ``span`` steps back, multiplied by ``A^span``, then squares the power) for the
forward, and the same scan with ``A^T`` run time-reversed for the adjoint
``G_t = A^T G_{t+1} + g_t`` with ``grad_A = sum_t G_t x_{t-1}^T`` and ``grad_x0 = A^T G_1``.

Used only by bench.py's ``cpu_baseline`` leg (timed on the host cores as the reference's own
CPU algorithm); the product path never imports it.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def _doubling(A: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """x_t = A x_{t-1} + v_t from a zero state, in ceil(log2 L) levels (dynonet/core.py:23-37)."""
    L = v.shape[-2]
    x = v.clone()
    power, span = A, 1
    while span < L:
        delayed = F.pad(x[..., : L - span, :], (0, 0, span, 0))
        x = x + delayed @ power.transpose(-1, -2)
        power = power @ power
        span *= 2
    return x


def linrec_forward(A: torch.Tensor, v: torch.Tensor, x0: torch.Tensor | None = None) -> torch.Tensor:
    """The forward op (dynonet/core.py:45-50): x0 folded into the first input, then the scan."""
    if x0 is not None and v.shape[-2] > 0:
        v = v.clone()
        v[..., 0, :] += (A @ x0.unsqueeze(-1)).squeeze(-1)
    return _doubling(A, v)


def linrec_backward(g: torch.Tensor, A: torch.Tensor, out: torch.Tensor, x0: torch.Tensor | None = None):
    """The adjoint op (dynonet/core.py:58-67): ``(grad_A, grad_v, grad_x0)``."""
    G = _doubling(A.transpose(-1, -2), g.flip(-2)).flip(-2)
    prev = torch.cat(
        ((torch.zeros_like(out[..., :1, :]) if x0 is None else x0.unsqueeze(-2)), out[..., :-1, :]), dim=-2
    )
    grad_A = G.transpose(-1, -2) @ prev
    grad_x0 = None if x0 is None else (A.transpose(-1, -2) @ G[..., 0, :].unsqueeze(-1)).squeeze(-1)
    return grad_A, G, grad_x0


class LinRec(torch.autograd.Function):
    """Autograd wiring of the two ops above (the reference registers the same pair,
    dynonet/core.py:76-86), so a CPU baseline can time forward + backward through conv1d too."""

    @staticmethod
    def forward(ctx, A, v):
        out = linrec_forward(A, v)
        ctx.save_for_backward(A, out)
        return out

    @staticmethod
    def backward(ctx, g):
        A, out = ctx.saved_tensors
        grad_A, grad_v, _ = linrec_backward(g, A, out)
        return grad_A, grad_v


def causal_depthwise_silu(x, tail, weight, bias):
    """The reference's eager CPU conv path (tsfast/models/architectures/mamba/core.py:38-58):
    ``silu`` of a causal depthwise convolution written as ``K`` shifted multiply-adds in
    channel-last layout. x [B, L, D], tail [B, D, K-1], weight [D, 1, K], bias [D]."""
    L, K = x.shape[1], weight.shape[-1]
    taps = weight[:, 0]
    buf = torch.cat((tail.transpose(1, 2), x), dim=1)  # [B, K-1+L, D]
    acc = bias + taps[:, 0] * buf[:, :L]
    for k in range(1, K):
        acc = acc + taps[:, k] * buf[:, k : k + L]
    return F.silu(acc)
