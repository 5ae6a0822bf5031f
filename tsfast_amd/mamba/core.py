"""The conv and selective-SSM sections of a Mamba layer, with fused-kernel dispatch.

Counterparts of ``tsfast/models/architectures/mamba/core.py``: ``_fused_conv`` (``:27-35``) and
``_fused_ssm`` / ``MambaLayer._ssm`` (``:61-70``, ``:147-173``). The fused backends are resolved
through ``dispatch.resolve`` over ``_CONV_BACKENDS`` / ``_SSM_BACKENDS`` (the ``"hip"`` family for
``"cuda"`` tensors). When no backend serves the inputs:

* the conv runs as one grouped ``F.conv1d`` over ``cat(tail, x)`` in channel-first layout;
* the SSM runs in time slices sized to keep ``[B, T, D, N]`` temporaries near 2^24 elements:
  per slice it forms ``lam = exp(delta A)`` and the drive ``(delta u) B``, scans them from the
  carried state (``selective_recurrence``, or a per-step loop for ``backend="eager"``),
  contracts with ``C`` and gates, so memory does not grow with the sequence length.
"""

from __future__ import annotations

__all__ = ["mamba_conv", "mamba_ssm"]

import torch
import torch.nn.functional as F

from .. import blocked_scan
from ..dispatch import resolve
from ..scan import selective_recurrence
from . import conv_hip, mamba_hip

# Module objects, not import paths: this dispatch may run inside a compiled forward.
_CONV_BACKENDS = {"hip": conv_hip}
_SSM_BACKENDS = {"hip": mamba_hip}
_SSM_AUTO_ORDER = {"cuda": ("hip",)}

# elements of one slice's [B, T, D, N] temporaries in the unfused SSM path
_SLICE_ELEMS = 1 << 24


def _fused_conv(x, tail, weight, bias):
    """The fused causal conv + SiLU backend's output, or None when none serves the inputs."""
    order = ("hip",) if x.device.type == "cuda" else ()
    mod = resolve("mamba.conv", _CONV_BACKENDS, order, (x, tail, weight, bias))
    return None if mod is None else mod.run(x, tail, weight, bias)


def mamba_conv(x, tail, weight, bias, backend: str = "scan"):
    """The conv section of a Mamba layer: ``silu(causal depthwise conv(cat(tail, x)))``.

    Args:
        x: in_proj chunk ``[B, L, D]`` (any strides); tail: carried left context
            ``[B, D, K-1]``; weight: depthwise kernel ``[D, 1, K]``; bias: ``[D]`` or None.
        backend: ``"scan"`` (fused kernel when available) or ``"eager"``.

    Returns:
        ``[B, L, D]``.
    """
    if backend == "scan":
        fused = _fused_conv(x, tail, weight, bias)
        if fused is not None:
            return fused
    padded = torch.cat((tail, x.transpose(1, 2)), dim=2)  # [B, D, K-1+L]
    return F.silu(F.conv1d(padded, weight, bias, groups=weight.shape[0])).transpose(1, 2)


def _fused_ssm(draw, A, B_t, C_t, u, z, Dp, h0):
    """The fused SSM backend's ``(out, h_last)``, or None when none serves the inputs."""
    order = _SSM_AUTO_ORDER.get(draw.device.type, ())
    mod = resolve("mamba.ssm", _SSM_BACKENDS, order, (draw, A, B_t, C_t, u, z, Dp, h0))
    return None if mod is None else mod.run(draw, A, B_t, C_t, u, z, Dp, h0)


def _sliced_ssm(draw, A, B_t, C_t, u, z, Dp, h0, per_step: bool):
    """The SSM without a fused kernel, one time slice at a time (see the module docstring)."""
    Bsz, L, D = draw.shape
    N = A.shape[-1]
    span = max(1, min(max(L, 1), _SLICE_ELEMS // max(1, Bsz * D * N)))
    state = None if h0 is None else h0.reshape(Bsz, D * N)
    pieces = []
    for t0 in range(0, L, span):
        sl = slice(t0, t0 + span)
        delta = F.softplus(draw[:, sl])  # [B, T, D]
        lam = torch.exp(delta.unsqueeze(-1) * A).flatten(-2)  # [B, T, D*N]
        drive = ((delta * u[:, sl]).unsqueeze(-1) * B_t[:, sl].unsqueeze(-2)).flatten(-2)
        scan = blocked_scan.sequential if per_step else selective_recurrence
        h = scan(lam, drive, state)
        y = (h.unflatten(-1, (D, N)) * C_t[:, sl].unsqueeze(-2)).sum(-1)
        pieces.append((y + Dp * u[:, sl]) * F.silu(z[:, sl]))
        state = h[:, -1]
    out = torch.cat(pieces, dim=1) if pieces else draw.new_empty(Bsz, 0, D)
    if state is None:
        state = draw.new_zeros(Bsz, D * N, dtype=torch.promote_types(draw.dtype, A.dtype))
    return out, state


def mamba_ssm(draw, A, B_t, C_t, u, z, Dp, h0=None, backend: str = "scan"):
    """The scan section of a Mamba layer after its projections (``MambaLayer._ssm``).

    Args:
        draw: pre-softplus step sizes ``[B, L, D]``.
        A: state matrix ``[D, N]`` (negative real).
        B_t, C_t: input / output projections per step ``[B, L, N]``.
        u: convolved input ``[B, L, D]``; z: gate input ``[B, L, D]``; Dp: skip ``[D]``.
        h0: initial state ``[B, D, N]`` or None.
        backend: ``"scan"`` (fused kernel when available, else the sliced scan) or ``"eager"``
            (the sliced path with a per-step loop).

    Returns:
        ``(out [B, L, D], h_last [B, D * N])``.
    """
    if backend not in ("scan", "eager"):
        raise ValueError(f"unknown backend {backend!r}, expected 'scan' or 'eager'")
    if backend == "scan":
        fused = _fused_ssm(draw, A, B_t, C_t, u, z, Dp, h0)
        if fused is not None:
            out, h_last = fused
            return out, h_last.flatten(-2)
    return _sliced_ssm(draw, A, B_t, C_t, u, z, Dp, h0, per_step=backend == "eager")
