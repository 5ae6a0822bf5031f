"""HIP backend for the constant-matrix linear recurrence ``x_t = A x_{t-1} + v_t``, float32.

GPU path of ``linear_recurrence`` (``tsfast/models/architectures/dynonet/core.py:103-127``),
whose ops ``tsfast::linear_recurrence`` / ``linear_recurrence_bwd`` (``:45-73``) run a log-doubling
scan: here one single-pass look-back scan per direction (``csrc/linrec.hip``) reads the input once
and writes the states once. ``supports(A, v, x0)`` and ``run(A, v, x0) -> x``, differentiable in
``A``, ``v`` and ``x0`` through the ``tsfast_hip::linear_recurrence_hip`` /
``linear_recurrence_hip_bwd`` ops, whose adjoint is the reference's: ``G_t = A^T G_{t+1} + g_t``,
``grad_v = G``, ``grad_A = sum_t G_t x_{t-1}^T``, ``grad_x0 = A^T G_1``.

Shapes follow the reference: ``A [..., n, n]``, ``v [..., L, n]``, ``x0 [..., n]`` with common
leading dims (``linear_recurrence`` broadcasts them first); states ``x_1 .. x_L`` as ``[..., L, n]``.
float32, ``1 <= n <= 16`` (``n <= 4`` a single-pass look-back scan, ``5..8`` a two-pass scan with a
thread per lane and chunk, ``9..16`` a two-pass scan with a 16-thread group per lane and chunk).
"""

from __future__ import annotations

__all__ = ["supports", "run"]

import math

import torch

from .. import _lib

_MAX_N = 16
_MAX_WIDE_L = 65535 * 256  # two-pass path (n > 4): chunks of 256 steps, one grid row each


def supports(A: torch.Tensor, v: torch.Tensor, x0: torch.Tensor | None) -> str | None:
    """Reason this backend cannot handle the inputs, or None when it can."""
    if v.device.type != "cuda":
        return f"input on {v.device.type}, hip backend is GPU-only"
    if any(t is not None and t.dtype != torch.float32 for t in (A, v, x0)):
        return "needs float32 tensors"
    if any(t is not None and t.device != v.device for t in (A, x0)):
        return "inputs on different devices"
    if v.dim() < 2 or A.dim() < 2:
        return "expected A [..., n, n] and v [..., L, n]"
    n = v.shape[-1]
    if not 1 <= n <= _MAX_N:
        return f"state size n={n} outside the supported range [1, {_MAX_N}]"
    if n > 4 and v.shape[-2] > _MAX_WIDE_L:
        return f"sequence length {v.shape[-2]} above {_MAX_WIDE_L} for n > 4"
    lead = v.shape[:-2]
    if tuple(A.shape) != tuple(lead) + (n, n):
        return f"A.shape {tuple(A.shape)} != {tuple(lead) + (n, n)}"
    if x0 is not None and tuple(x0.shape) != tuple(lead) + (n,):
        return f"x0.shape {tuple(x0.shape)} != {tuple(lead) + (n,)}"
    return None


def _workspace(lib, lanes, L, n, device):
    nbytes = lib.tsfast_hip_linrec_workspace_bytes(lanes, L, n)
    if nbytes < 0:
        raise RuntimeError("tsfast_hip_linrec_workspace_bytes: unsupported shape")
    return _lib.workspace(nbytes, device), nbytes


@torch.library.custom_op("tsfast_hip::linear_recurrence_hip", mutates_args=())
def _linrec_op(A: torch.Tensor, v: torch.Tensor, x0: torch.Tensor | None) -> torch.Tensor:
    lib = _lib.load()
    _lib.sync_deterministic()
    A, v = A.contiguous(), v.contiguous()
    x0 = x0.contiguous() if x0 is not None else None
    for name, t in (("A", A), ("v", v), ("x0", x0)):
        _lib.require(t, name, (torch.float32,), v.device)
    lanes, L, n = v.shape
    x = torch.empty_like(v)
    ws, nbytes = _workspace(lib, lanes, L, n, v.device)
    _lib.check(
        lib.tsfast_hip_linrec_fwd(
            lanes, L, n, _lib.ptr(A), _lib.ptr(v), _lib.ptr(x0), _lib.ptr(x), _lib.ptr(ws), nbytes, _lib.stream_of(v)
        ),
        "tsfast_hip_linrec_fwd",
    )
    if n <= 4:  # the single-pass look-back path (n = 5..8 run two passes, no look-back)
        _lib.check_lookback(ws, "tsfast_hip_linrec_fwd")
    return x


@_linrec_op.register_fake
def _(A, v, x0):
    return torch.empty_like(v)


@torch.library.custom_op("tsfast_hip::linear_recurrence_hip_bwd", mutates_args=())
def _linrec_bwd_op(
    g: torch.Tensor, A: torch.Tensor, out: torch.Tensor, x0: torch.Tensor | None
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    lib = _lib.load()
    _lib.sync_deterministic()
    g, A, out = g.contiguous(), A.contiguous(), out.contiguous()
    x0 = x0.contiguous() if x0 is not None else None
    for name, t in (("g", g), ("A", A), ("out", out), ("x0", x0)):
        _lib.require(t, name, (torch.float32,), out.device)
    lanes, L, n = out.shape
    gA = torch.empty_like(A)
    gv = torch.empty_like(g)
    gx0 = torch.empty_like(x0) if x0 is not None else None
    ws, nbytes = _workspace(lib, lanes, L, n, out.device)
    _lib.check(
        lib.tsfast_hip_linrec_bwd(
            lanes, L, n, _lib.ptr(g), _lib.ptr(A), _lib.ptr(out), _lib.ptr(x0), _lib.ptr(gA), _lib.ptr(gv),
            _lib.ptr(gx0), _lib.ptr(ws), nbytes, _lib.stream_of(out),
        ),
        "tsfast_hip_linrec_bwd",
    )
    if n <= 4:  # the single-pass look-back path (n = 5..8 run two passes, no look-back)
        _lib.check_lookback(ws, "tsfast_hip_linrec_bwd")
    return gA, gv, (gx0 if gx0 is not None else A.new_empty(0))


@_linrec_bwd_op.register_fake
def _(g, A, out, x0):
    gx0 = torch.empty_like(x0) if x0 is not None else A.new_empty(0)
    return torch.empty_like(A), torch.empty_like(g), gx0


def _linrec_setup(ctx, inputs, output):
    A, v, x0 = inputs
    ctx.save_for_backward(A, output, x0)


def _linrec_backward(ctx, g):
    A, out, x0 = ctx.saved_tensors
    grad_A, grad_v, grad_x0 = _linrec_bwd_op(g, A, out, x0)
    return grad_A, grad_v, (grad_x0 if x0 is not None else None)


_linrec_op.register_autograd(_linrec_backward, setup_context=_linrec_setup)


def run(A: torch.Tensor, v: torch.Tensor, x0: torch.Tensor | None) -> torch.Tensor:
    """States ``x_1 .. x_L`` of ``x_t = A x_{t-1} + v_t`` (``[..., L, n]``). The leading dims are
    flattened to lanes outside the op, so autograd carries lane gradients back to the callers'
    (possibly broadcast) tensors."""
    L, n = v.shape[-2], v.shape[-1]
    lanes = math.prod(v.shape[:-2])
    A_lane = A.reshape(lanes, n, n)
    v_lane = v.reshape(lanes, L, n)
    x0_lane = x0.reshape(lanes, n) if x0 is not None else None
    return _linrec_op(A_lane, v_lane, x0_lane).reshape(v.shape)
