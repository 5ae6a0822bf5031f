"""HIP backend for banks of scalar all-pole (order-na IIR) recurrences, float32.

Computes ``y_t = w_t - sum_{i=1..na} a_i y_{t-i}`` per lane — the denominator of the dynoNet
G-block. Drop-in for the ``dynonet.allpole`` registry of
``tsfast/models/architectures/dynonet/core.py:20`` (the role of ``allpole_triton.py``):
``supports(a, w, y0)`` and ``run(a, w, y0) -> y``, differentiable in ``a``, ``w`` and ``y0``
through the ``tsfast_hip::dynonet_allpole`` / ``dynonet_allpole_bwd`` ops. ``y0`` holds the
outputs before the sequence, newest first (``y0[..., j] = y_{-1-j}``).

The kernels (``csrc/allpole.hip``) are specialised per order ``1 <= na <= 16`` at build time
and split time into chunks joined through the companion-matrix power; the backward's y0 head
taps and ``grad_y0`` are computed on the device as well.
"""

from __future__ import annotations

__all__ = ["supports", "run"]

import torch

from .. import _lib

_MAX_NA = 16
_LB_NA = 4  # highest order on the single-pass look-back path (allpole_core.h kLbNA)


def supports(a: torch.Tensor, w: torch.Tensor, y0: torch.Tensor | None) -> str | None:
    """Reason this backend cannot handle the inputs, or None when it can."""
    if w.device.type != "cuda":
        return f"input on {w.device.type}, hip backend is GPU-only"
    if any(t is not None and t.dtype != torch.float32 for t in (a, w, y0)):
        return "needs float32 tensors"
    if any(t is not None and t.device != w.device for t in (a, y0)):
        return "inputs on different devices"
    if w.dim() < 2:
        return "w must have at least a batch and a time axis"
    na = a.shape[-1]
    if not 1 <= na <= _MAX_NA:
        return f"na={na} outside the supported range [1, {_MAX_NA}]"
    lead = w.shape[:-1]
    try:
        if torch.broadcast_shapes(a.shape[:-1], lead) != lead:
            return f"a leading dims {tuple(a.shape[:-1])} do not broadcast into {tuple(lead)}"
        if y0 is not None and torch.broadcast_shapes(y0.shape[:-1], lead) != lead:
            return f"y0 leading dims {tuple(y0.shape[:-1])} do not broadcast into {tuple(lead)}"
    except RuntimeError as e:
        return f"shape mismatch: {e}"
    if y0 is not None and y0.shape[-1] != na:
        return f"y0 state dim {y0.shape[-1]} != na {na}"
    return None


@torch.library.custom_op("tsfast_hip::dynonet_allpole", mutates_args=())
def _allpole_op(a: torch.Tensor, w: torch.Tensor, y0: torch.Tensor | None) -> torch.Tensor:
    lib = _lib.load()
    _lib.sync_deterministic()
    a, w = a.contiguous(), w.contiguous()
    y0 = y0.contiguous() if y0 is not None else None
    for name, t in (("a", a), ("w", w), ("y0", y0)):
        _lib.require(t, name, (torch.float32,), w.device)
    lanes, L = w.shape
    na = a.shape[-1]
    y = torch.empty_like(w)
    nbytes = lib.tsfast_hip_allpole_workspace_bytes(lanes, L, na)
    ws = _lib.workspace(nbytes, w.device)
    _lib.check(
        lib.tsfast_hip_allpole_fwd(
            lanes, L, na, _lib.ptr(a), _lib.ptr(w), _lib.ptr(y0), _lib.ptr(y), _lib.ptr(ws), nbytes, _lib.stream_of(w)
        ),
        "tsfast_hip_allpole_fwd",
    )
    if na <= _LB_NA:  # the single-pass look-back path (higher orders run two passes, no look-back)
        _lib.check_lookback(ws, "tsfast_hip_allpole_fwd")
    return y


@_allpole_op.register_fake
def _(a, w, y0):
    return torch.empty_like(w)


@torch.library.custom_op("tsfast_hip::dynonet_allpole_bwd", mutates_args=())
def _allpole_bwd_op(
    g: torch.Tensor, a: torch.Tensor, y: torch.Tensor, y0: torch.Tensor | None
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    lib = _lib.load()
    _lib.sync_deterministic()
    g, a, y = g.contiguous(), a.contiguous(), y.contiguous()
    y0 = y0.contiguous() if y0 is not None else None
    for name, t in (("g", g), ("a", a), ("y", y), ("y0", y0)):
        _lib.require(t, name, (torch.float32,), y.device)
    lanes, L = y.shape
    na = a.shape[-1]
    gw = torch.empty_like(g)
    ga = torch.empty_like(a)
    gy0 = torch.empty_like(y0) if y0 is not None else None
    nbytes = lib.tsfast_hip_allpole_workspace_bytes(lanes, L, na)
    ws = _lib.workspace(nbytes, y.device)
    _lib.check(
        lib.tsfast_hip_allpole_bwd(
            lanes, L, na, _lib.ptr(g), _lib.ptr(a), _lib.ptr(y), _lib.ptr(y0), _lib.ptr(gw), _lib.ptr(ga),
            _lib.ptr(gy0), _lib.ptr(ws), nbytes, _lib.stream_of(y),
        ),
        "tsfast_hip_allpole_bwd",
    )
    if na <= _LB_NA:  # the single-pass look-back path (higher orders run two passes, no look-back)
        _lib.check_lookback(ws, "tsfast_hip_allpole_bwd")
    return ga, gw, (gy0 if gy0 is not None else a.new_empty(0))


@_allpole_bwd_op.register_fake
def _(g, a, y, y0):
    gy0 = torch.empty_like(y0) if y0 is not None else a.new_empty(0)
    return torch.empty_like(a), torch.empty_like(g), gy0


def _allpole_setup(ctx, inputs, output):
    a, w, y0 = inputs
    ctx.save_for_backward(a, output, y0)


def _allpole_backward(ctx, g):
    a, y, y0 = ctx.saved_tensors
    grad_a, grad_w, grad_y0 = _allpole_bwd_op(g, a, y, y0)
    return grad_a, grad_w, (grad_y0 if y0 is not None else None)


_allpole_op.register_autograd(_allpole_backward, setup_context=_allpole_setup)


def run(a: torch.Tensor, w: torch.Tensor, y0: torch.Tensor | None) -> torch.Tensor:
    """Run the filter bank; broadcasts ``a``/``y0`` over ``w``'s leading dims and flattens to lanes
    outside the op, so autograd reduces lane gradients to the callers' shapes (``allpole_triton.py:236-247``)."""
    lead, L, na = w.shape[:-1], w.shape[-1], a.shape[-1]
    a_lane = a.broadcast_to(lead + (na,)).reshape(-1, na)
    w_flat = w.reshape(-1, L)
    y0_lane = y0.broadcast_to(lead + (na,)).reshape(-1, na) if y0 is not None else None
    return _allpole_op(a_lane, w_flat, y0_lane).reshape(w.shape)
