"""dynoNet sections with fused-kernel dispatch, and the constant-matrix recurrence.

Counterparts of ``tsfast/models/architectures/dynonet/core.py``:

* ``linear_recurrence`` (``:103-127``): ``x_t = A x_{t-1} + v_t`` with constant ``A [..., n, n]``
  and its matrix adjoint. On GPU the ``"hip"`` family serves state sizes n <= 16 (a single-pass
  scan for n <= 4, two-pass scans above); otherwise the ``tsfast_hip::linear_recurrence`` op
  runs the blocked torch scan of :mod:`tsfast_amd.blocked_scan` (the reference runs a
  log-doubling scan, ``:23-37``).
* ``allpole``: the all-pole branch of ``LinearDynamicalOperator.forward`` (``:221-248``), the
  fused backend when one serves the inputs (``_fused_allpole``, ``:91-100``), else
  ``linear_recurrence`` over the companion matrices.
* ``linear_dynamical_operator``: the whole G-block (FIR, all-pole, sum over inputs), fused
  when a backend serves it.

Adjoint of the matrix recurrence: ``G_t = A^T G_{t+1} + g_t``, ``dL/dv = G``,
``dL/dA = sum_t G_t x_{t-1}^T``, ``dL/dx_0 = A^T G_1``.
"""

from __future__ import annotations

__all__ = ["linear_recurrence", "allpole", "companion", "linear_dynamical_operator"]

import torch
import torch.nn.functional as F

from .. import blocked_scan
from ..dispatch import resolve
from . import allpole_hip, gblock_hip, linrec_hip

_ALLPOLE_BACKENDS = {"hip": allpole_hip}
_GBLOCK_BACKENDS = {"hip": gblock_hip}
_LINREC_BACKENDS = {"hip": linrec_hip}


@torch.library.custom_op("tsfast_hip::linear_recurrence", mutates_args=())
def _linear_recurrence_op(A: torch.Tensor, v: torch.Tensor, x0: torch.Tensor | None) -> torch.Tensor:
    return blocked_scan.scan_matrix(A, v, x0)


@_linear_recurrence_op.register_fake
def _(A, v, x0):
    return torch.empty_like(v)


@torch.library.custom_op("tsfast_hip::linear_recurrence_bwd", mutates_args=())
def _linear_recurrence_bwd_op(
    g: torch.Tensor, A: torch.Tensor, out: torch.Tensor, x0: torch.Tensor | None
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    At = A.transpose(-1, -2)
    G = blocked_scan.scan_matrix(At, g.flip(-2)).flip(-2)  # reverse-time scan with A^T
    prev = out.roll(1, dims=-2)  # x_{t-1} for every step t
    if prev.shape[-2] > 0:
        prev[..., 0, :] = 0 if x0 is None else x0
    grad_A = torch.einsum("...ti,...tj->...ij", G, prev)
    if x0 is None:
        grad_x0 = A.new_empty(0)
    elif G.shape[-2] > 0:
        grad_x0 = (At @ G[..., 0, :].unsqueeze(-1)).squeeze(-1)
    else:
        grad_x0 = torch.zeros_like(x0)
    return grad_A, G, grad_x0


@_linear_recurrence_bwd_op.register_fake
def _(g, A, out, x0):
    return torch.empty_like(A), torch.empty_like(g), (A.new_empty(0) if x0 is None else torch.empty_like(x0))


def _linrec_save(ctx, inputs, output):
    A, _, x0 = inputs
    ctx.save_for_backward(A, output, x0)


def _linrec_grads(ctx, g):
    A, out, x0 = ctx.saved_tensors
    gA, gv, gx0 = _linear_recurrence_bwd_op(g, A, out, x0)
    return gA, gv, None if x0 is None else gx0


_linear_recurrence_op.register_autograd(_linrec_grads, setup_context=_linrec_save)


def linear_recurrence(A: torch.Tensor, v: torch.Tensor, x0: torch.Tensor | None = None) -> torch.Tensor:
    """``x_t = A x_{t-1} + v_t`` with constant ``A [..., n, n]`` (``dynonet/core.py:103-127``).

    ``A``, ``v [..., L, n]`` and ``x0 [..., n]`` (zero if None) are broadcast to common leading
    dims; a backend that serves them (the ``"hip"`` family for ``"cuda"`` tensors) runs the
    scan, else the ``tsfast_hip::linear_recurrence`` op. Returns ``x_1 .. x_L``, ``[..., L, n]``.
    """
    lead = torch.broadcast_shapes(A.shape[:-2], v.shape[:-2], () if x0 is None else x0.shape[:-1])
    args = (
        A.expand(*lead, *A.shape[-2:]),
        v.expand(*lead, *v.shape[-2:]),
        None if x0 is None else x0.expand(*lead, x0.shape[-1]),
    )
    order = ("hip",) if v.device.type == "cuda" else ()
    mod = resolve("dynonet.linear_recurrence", _LINREC_BACKENDS, order, args)
    return mod.run(*args) if mod is not None else _linear_recurrence_op(*args)


def companion(a: torch.Tensor) -> torch.Tensor:
    """Companion matrices ``[..., na, na]`` of monic denominators ``1 + a_1 q^-1 + ... + a_na q^-na``:
    first row ``-a``, then the unit shift (``LinearDynamicalOperator._companion``, ``core.py:186-190``)."""
    na = a.shape[-1]
    shift = torch.eye(na, dtype=a.dtype, device=a.device)[:-1].expand(*a.shape[:-1], na - 1, na)
    return torch.cat((-a.unsqueeze(-2), shift), dim=-2)


def _fused_allpole(a, w, y0):
    """The fused all-pole backend's output, or None when none serves the inputs."""
    order = ("hip",) if w.device.type == "cuda" else ()
    mod = resolve("dynonet.allpole", _ALLPOLE_BACKENDS, order, (a, w, y0))
    return None if mod is None else mod.run(a, w, y0)


def allpole(a: torch.Tensor, w: torch.Tensor, y0: torch.Tensor | None = None) -> torch.Tensor:
    """``y_t = w_t - sum_i a_i y_{t-i}`` over lanes ``w [..., L]`` with ``a [..., na]``, ``y0 [..., na]``.

    The fused kernel when one serves the inputs, else ``linear_recurrence`` over the companion
    matrices: the companion state is a shift register of past outputs, so ``y`` is its first
    component.
    """
    y = _fused_allpole(a, w, y0)
    if y is not None:
        return y
    na = a.shape[-1]
    x = linear_recurrence(companion(a), F.pad(w.unsqueeze(-1), (0, na - 1)), y0)
    return x[..., 0]


def linear_dynamical_operator(
    u: torch.Tensor,
    b_coeff: torch.Tensor,
    a_coeff: torch.Tensor,
    state: dict | None = None,
    return_state: bool = False,
) -> torch.Tensor | tuple[torch.Tensor, dict]:
    """The body of ``LinearDynamicalOperator.forward`` (dynonet/core.py:196-258) for ``na >= 1``.

    ``u [B, L, I]``, ``b_coeff [O, I, nb]``, ``a_coeff [O, I, na]``; ``state`` is the reference's
    ``{"u": FIR tail [B, nb-1, I], "x": IIR states [B, I*O, na]}`` (zeros if None). The fused
    G-block backend runs FIR, all-pole and the sum over inputs when it serves the inputs (one
    pass for na <= 4, this library's FIR and all-pole ops for higher orders); otherwise the
    reference's three stages run (grouped ``conv1d`` with flipped taps, the all-pole op per pair,
    the sum over inputs). Returns ``y [B, L, O]`` and, with
    ``return_state``, the new state.
    """
    B, L, I = u.shape
    O, _, nb = b_coeff.shape
    na = a_coeff.shape[-1]
    P = I * O
    # plain branches, not a mapping `match`: Dynamo cannot trace mapping patterns
    if state is None:
        u_tail = u.new_zeros(B, nb - 1, I)
        x0 = u.new_zeros(B, P, na)
    elif isinstance(state, dict) and "u" in state and "x" in state:
        u_tail, x0 = state["u"], state["x"]
    else:
        raise TypeError(f"expected state dict {{'u': tensor, 'x': tensor}}, got {type(state)}")
    order = ("hip",) if u.device.type == "cuda" else ()
    mod = resolve("dynonet.gblock", _GBLOCK_BACKENDS, order, (u, b_coeff, a_coeff, u_tail, x0))
    if mod is not None:
        y, x_last = mod.run(u, b_coeff, a_coeff, u_tail, x0)
    else:
        u_buf = torch.cat((u_tail, u), dim=1)
        weight = b_coeff.permute(1, 0, 2).reshape(P, 1, nb).flip(-1)
        w = F.conv1d(u_buf.transpose(1, 2), weight, groups=I)
        a_pairs = a_coeff.permute(1, 0, 2).reshape(P, na).expand(B, P, na)
        y_pairs = allpole(a_pairs, w, x0)
        x_last = (
            y_pairs[..., L - na :].flip(-1) if L >= na else torch.cat((y_pairs.flip(-1), x0[..., : na - L]), dim=-1)
        )
        y = y_pairs.view(B, I, O, L).sum(1).transpose(1, 2)
    if not return_state:
        return y
    u_buf = torch.cat((u_tail, u), dim=1)
    return y, {"u": u_buf[:, u_buf.shape[1] - (nb - 1) :], "x": x_last}
