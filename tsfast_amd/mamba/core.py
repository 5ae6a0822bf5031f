"""The Mamba conv and selective-SSM sections with their fused-kernel dispatch.

Mirrors ``tsfast/models/architectures/mamba/core.py``: ``_fused_conv`` /
``_causal_depthwise_silu`` (``:27-58``) and ``MambaLayer._ssm`` / ``_fused_ssm`` (``:61-70``,
``:147-173``). Fused backends are resolved through ``dispatch.resolve`` over ``_CONV_BACKENDS``
and ``_SSM_BACKENDS`` (here the ``"hip"`` family first for ``"cuda"`` tensors); when none serves
the inputs, the conv runs as shifted multiply-adds and the SSM generic path materialises
``lam = exp(delta A)`` and ``v = (delta u) B`` and runs ``selective_recurrence`` followed by the
C contraction.
"""

from __future__ import annotations

__all__ = ["mamba_conv", "mamba_ssm"]

import torch
import torch.nn.functional as F

from ..dispatch import resolve
from ..scan import _diagonal_recurrence_sequential, selective_recurrence
from . import conv_hip, mamba_hip

# Module objects, not import paths: this dispatch may run inside a compiled forward.
_CONV_BACKENDS = {"hip": conv_hip}
_SSM_BACKENDS = {"hip": mamba_hip}
_SSM_AUTO_ORDER = {"cuda": ("hip",)}


def _fused_conv(x, tail, weight, bias):
    """Dispatch the fused causal conv + SiLU kernel; None means run the eager conv path."""
    order = ("hip",) if x.device.type == "cuda" else ()
    mod = resolve("mamba.conv", _CONV_BACKENDS, order, (x, tail, weight, bias))
    return None if mod is None else mod.run(x, tail, weight, bias)


def _causal_depthwise_silu(x, tail, weight, bias):
    """Causal depthwise convolution + SiLU as ``K`` shifted multiply-adds, channel-last:
    x [B, L, D], tail [B, D, K-1], weight [D, 1, K], bias [D] or None."""
    L, w = x.shape[1], weight[:, 0]
    buf = torch.cat((tail.mT, x), dim=1)
    y = w[:, 0] * buf[:, :L]
    if bias is not None:
        y = y + bias
    for i in range(1, weight.shape[-1]):
        y = y + w[:, i] * buf[:, i : i + L]
    return F.silu(y)


def mamba_conv(x, tail, weight, bias, backend: str = "scan"):
    """The conv section of ``MambaLayer.forward``: ``silu(conv1d(cat(tail, x)))`` per channel.

    Args:
        x: in_proj chunk ``[B, L, D]`` (any strides); tail: carried left context
            ``[B, D, K-1]``; weight: depthwise kernel ``[D, 1, K]``; bias: ``[D]`` or None.
        backend: ``"scan"`` (fused kernel when available) or ``"eager"``.
    """
    if backend == "scan":
        fused = _fused_conv(x, tail, weight, bias)
        if fused is not None:
            return fused
    return _causal_depthwise_silu(x, tail, weight, bias)


def _fused_ssm(draw, A, B_t, C_t, u, z, Dp, h0):
    """Dispatch the fused SSM kernel; None means run the generic scan path."""
    order = _SSM_AUTO_ORDER.get(draw.device.type, ())
    mod = resolve("mamba.ssm", _SSM_BACKENDS, order, (draw, A, B_t, C_t, u, z, Dp, h0))
    return None if mod is None else mod.run(draw, A, B_t, C_t, u, z, Dp, h0)


def mamba_ssm(draw, A, B_t, C_t, u, z, Dp, h0=None, backend: str = "scan"):
    """The scan section of ``MambaLayer._ssm`` after the projections.

    Args:
        draw: pre-softplus step sizes ``[B, L, D]``.
        A: state matrix ``[D, N]`` (negative real).
        B_t, C_t: input / output projections per step ``[B, L, N]``.
        u: convolved input ``[B, L, D]``; z: gate input ``[B, L, D]``; Dp: skip ``[D]``.
        h0: initial state ``[B, D, N]`` or None.
        backend: ``"scan"`` (fused kernel when available, else the parallel scan) or ``"eager"``.

    Returns:
        ``(out [B, L, D], h_last [B, D * N])``.
    """
    B_sz, L, D = draw.shape
    N = A.shape[-1]
    if backend == "scan":
        fused = _fused_ssm(draw, A, B_t, C_t, u, z, Dp, h0)
        if fused is not None:
            out, h_last = fused
            return out, h_last.flatten(-2)
    delta = F.softplus(draw)
    lam = torch.exp(delta.unsqueeze(-1) * A)
    v = (delta * u).unsqueeze(-1) * B_t.unsqueeze(-2)
    h0_flat = h0.reshape(B_sz, D * N) if h0 is not None else None
    if backend == "scan":
        h = selective_recurrence(lam.flatten(-2), v.flatten(-2), h0_flat)
    elif backend == "eager":
        h = _diagonal_recurrence_sequential(lam.flatten(-2), v.flatten(-2), h0_flat)
    else:
        raise ValueError(f"unknown backend {backend!r}, expected 'scan' or 'eager'")
    y = (h.view(B_sz, L, D, N) * C_t.unsqueeze(-2)).sum(-1)
    return (y + Dp * u) * F.silu(z), h[..., -1, :]
